// LDS tile staging shared by the prefill-shaped kernels.
//
// A "64-row tile" is rows [row0, row0 + 64) of a row-major [rows, D] matrix.
// It can be staged two ways:
//  * natural, row-permuted (pitch D*sizeof(T) + 16 bytes): tile row r lands
//    at LDS row perm_row(r), so that a 32x32 MFMA whose A operand reads LDS
//    rows 32t + (lane % 32) produces, in lane half hh / accumulator register
//    reg, the tile row 32hh + 16t + reg;
//  * transposed (pitch 64*sizeof(T) + 16 bytes): LDS row d holds column d of
//    the tile with the 64 tile rows contiguous, which is the layout an MFMA
//    operand needs when the product contracts over the tile rows.
// Rows at or past `limit` are written as zeros and never read from memory.
#pragma once

#include "pf_common.hpp"

namespace pf {

__device__ inline int perm_row(int r) {
  return ((r >> 4) & 1) * 32 + ((r >> 2) & 3) * 8 + (r >> 5) * 4 + (r & 3);
}

template <typename T, int D>
struct TileGeom {
  static constexpr int ES = sizeof(T);
  static constexpr int EPC = 16 / ES;           // elements per 16-byte chunk
  static constexpr int NDC = D / EPC;           // chunks per row
  static constexpr int NAT_PITCH = D * ES + 16; // natural layout row pitch
  static constexpr int TRN_PITCH = 64 * ES + 16;
  static constexpr int NAT_BYTES = 64 * NAT_PITCH;
  static constexpr int TRN_BYTES = D * TRN_PITCH;
  static constexpr int ITEMS = 16 * NDC;        // (4-row group, chunk) items
};

// Stage a 64-row tile with all 256 threads of a workgroup. `src` points at
// row 0 of the matrix (row stride D). Writes the natural (permuted) copy to
// `nat` and/or the transposed copy to `trn` (either may be null).
template <typename T, int D>
__device__ inline void stage_tile(const T* src, int row0, int limit, char* nat, char* trn, int tid) {
  using G = TileGeom<T, D>;
#pragma unroll
  for (int u = 0; u < (G::ITEMS + 255) / 256; ++u) {
    const int c = tid + 256 * u;
    if (G::ITEMS % 256 != 0 && c >= G::ITEMS) break;
    const int kg = c & 15, dc = c >> 4;
    u32x4 ch[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = row0 + 4 * kg + r;
      ch[r] = (row < limit) ? ldg16(src + (int64_t)row * D + dc * G::EPC) : (u32x4){0u, 0u, 0u, 0u};
    }
    if (nat != nullptr) {
#pragma unroll
      for (int r = 0; r < 4; ++r) sts16(nat + perm_row(4 * kg + r) * G::NAT_PITCH + dc * 16, ch[r]);
    }
    if (trn != nullptr) {
      if constexpr (G::ES == 4) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const u32x4 o4 = {ch[0][e], ch[1][e], ch[2][e], ch[3][e]};
          sts16(trn + (dc * 4 + e) * G::TRN_PITCH + kg * 16, o4);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int wd = e >> 1, sh = (e & 1) * 16;
          const uint32_t v0 = (ch[0][wd] >> sh) & 0xffffu, v1 = (ch[1][wd] >> sh) & 0xffffu;
          const uint32_t v2 = (ch[2][wd] >> sh) & 0xffffu, v3 = (ch[3][wd] >> sh) & 0xffffu;
          const u32x2 o2 = {v0 | (v1 << 16), v2 | (v3 << 16)};
          *reinterpret_cast<u32x2*>(trn + (dc * 8 + e) * G::TRN_PITCH + kg * 8) = o2;
        }
      }
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

// acc(32x32 tiles t=0,1) += A rows from a natural-permuted LDS tile x B frags
// (contraction over D): the "S^T = K Q^T" step.
template <typename T, int D>
__device__ inline void mfma_rows_x_frags(const char* nat, int l32, int hh,
                                         const typename Mfma32<T>::Frag* bf, f32x16& s0, f32x16& s1) {
  using MF = Mfma32<T>;
  using G = TileGeom<T, D>;
  constexpr int FPC = frags_per_chunk<T>();
  const char* r0 = nat + l32 * G::NAT_PITCH + hh * (D / 2) * G::ES;
  const char* r1 = nat + (32 + l32) * G::NAT_PITCH + hh * (D / 2) * G::ES;
#pragma unroll
  for (int c = 0; c < D / 2 / G::EPC; ++c) {
    const u32x4 a0 = lds16(r0 + c * 16);
    const u32x4 a1 = lds16(r1 + c * 16);
#pragma unroll
    for (int f = 0; f < FPC; ++f) {
      s0 = MF::run(chunk_frag<T>(a0, f), bf[c * FPC + f], s0);
      s1 = MF::run(chunk_frag<T>(a1, f), bf[c * FPC + f], s1);
    }
  }
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

// acc[dt] += A rows of a transposed LDS tile (row 32dt + l32, this lane half's
// 32 contiguous tile rows) x packed B frags: the "O^T += V^T P^T" step.
template <typename T, int D>
__device__ inline void mfma_trn_x_frags(const char* trn, int l32, int hh,
                                        const typename Mfma32<T>::Frag* bf, f32x16* acc) {
  using MF = Mfma32<T>;
  using G = TileGeom<T, D>;
  constexpr int FPC = frags_per_chunk<T>();
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) {
    const char* r = trn + (32 * dt + l32) * G::TRN_PITCH + hh * 32 * G::ES;
#pragma unroll
    for (int c = 0; c < 32 * G::ES / 16; ++c) {
      const u32x4 a = lds16(r + c * 16);
#pragma unroll
      for (int f = 0; f < FPC; ++f) acc[dt] = MF::run(chunk_frag<T>(a, f), bf[c * FPC + f], acc[dt]);
    }
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
