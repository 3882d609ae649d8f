// Forward prefill attention for gfx950 (CDNA4), with optional fused RoPE.
//
// Replaces the reference's `flash_attention_fwd` pallas_call
// (flash_attention.py:162-227, kernel :61-159) and `flash_attention_rope_fwd`
// (fused_rope.py:183-213, kernel :53-113).
//
// Work decomposition: one workgroup of 4 waves per (batch, query head, 128-row
// query block); each wave owns 32 query rows. The grid is 1-D: heavy (late)
// query blocks first for causal load balance, and the query heads of one GQA
// group on one XCD so they share K/V in that XCD's L2 (see xcd_remap).
//
// Per 64-key block the workgroup stages K and V in LDS, double-buffered: the
// global loads for block j+1 are in flight while block j is computed, and one
// barrier per block separates the two buffers.
//   S^T = K . Q^T   (A = K rows from LDS, B = Q held in registers)
//   O^T += V^T . P^T (A = V^T fragments from LDS, B = P from the S^T accumulators)
// With S^T, lane l owns query l%32: the online-softmax row statistics are
// in-lane except one exchange between the two lane halves. K rows are stored
// in LDS in a permuted order so that lane half hh's 32 accumulator values are
// keys [32hh, 32hh+32) of the block, exactly the k-slots the P^T operand
// needs -- P never moves between lanes.
// V^T fragments: for 16-bit types V stays row-major in LDS and is read with
// the gfx950 transposing LDS load (ds_read_b64_tr_b16: within each 16-lane
// group, lane i receives element [4t + i/4][i%4] of the 16 x 4 block the group
// addressed, so lane j pointing at V[k0 + j/4][d0 + 4(j%4)] hands lane i the
// values V[k0 + t][d0 + i]). For float32 V is staged transposed.
// LDS tiles are unpadded with 16-byte chunks XOR-swizzled per row so the MFMA
// reads and the staging writes are free of bank conflicts.
//
// Semantics (flash_attention.py): mask k >= kv_len and (causal) k > q, with
// K/V rows past kv_len never read (zero-filled) (:95-120); online softmax in
// float32 (:123-134); whole-tile skipping (:136-147); o = acc / l with l == 0
// giving o = 0 and lse = 0 (:150-159); lse is the natural log-sum-exp of the
// scaled scores. Scores are kept in the log2 domain (exp2 with log2(e) folded
// into the scale) and converted back for the LSE.
#include "pf_common.hpp"
#include "pf_kernels.hpp"
#include "pf_tiles.hpp"

namespace pf {

namespace {

constexpr int kFwdBM = 128;  // query rows per workgroup
constexpr int kFwdBN = 64;   // keys per block

template <typename T, int D, bool ROPE>
struct FwdTiles {
  static constexpr int ES = sizeof(T);
  static constexpr int EPC = 16 / ES;         // elements per 16-byte chunk
  static constexpr int CPR = D / EPC;         // chunks per row
  static constexpr bool TR = (ES == 2);       // transposing LDS reads for V
  static constexpr int K_BYTES = kFwdBN * D * ES;
  static constexpr int VT_PITCH = kFwdBN * ES + 16;
  static constexpr int V_BYTES = TR ? kFwdBN * D * ES : D * VT_PITCH;
  static constexpr int K_ITEMS = ROPE ? kFwdBN * CPR / 2 : kFwdBN * CPR;   // per block
  static constexpr int K_PER_T = (K_ITEMS + 255) / 256;
  static constexpr int K_CHUNKS = ROPE ? 2 : 1;                             // chunks per item
  static constexpr int V_ITEMS = TR ? kFwdBN * CPR : 16 * CPR;              // f32: 4-row groups
  static constexpr int V_PER_T = (V_ITEMS + 255) / 256;
  static constexpr int V_CHUNKS = TR ? 1 : 4;
  // 16-byte chunk swizzles (row-dependent XOR keeps each row's chunks in place)
  __device__ static int kswz(int row) { return row & (CPR >= 16 ? 15 : CPR - 1); }
  __device__ static int vswz(int row) { return CPR >= 16 ? 4 * (row & 3) : 4 * (row & 1); }
};

template <typename T, int D, bool CAUSAL, bool ROPE>
__global__ __launch_bounds__(256, (sizeof(T) == 4 && D == 128) ? 1 : 2) void pf_attn_fwd_kernel(FwdParams p) {
  using MF = Mfma32<T>;
  using Frag = typename MF::Frag;
  using G = FwdTiles<T, D, ROPE>;
  constexpr int BM = kFwdBM, BN = kFwdBN;
  constexpr int HALF = D / 2;
  constexpr int ES = G::ES, EPC = G::EPC, CPR = G::CPR;
  constexpr int FPC = frags_per_chunk<T>();
  constexpr int QF = HALF / MF::kK;  // Q fragments per lane
  constexpr int NDT = D / 32;        // 32-row tiles of O^T
  constexpr int PF = 32 / MF::kK;    // P fragments per lane per block

  __shared__ __attribute__((aligned(16))) char smem[2 * (G::K_BYTES + G::V_BYTES)];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int hh = lane >> 5;
  const int l32 = lane & 31;

  const int w = xcd_remap(blockIdx.x, p.n_work, p.g);
  const int member = w % p.g;
  int rest = w / p.g;
  const int kvh = rest % p.Hkv;
  rest /= p.Hkv;
  const int b = rest % p.B;
  const int qblk = p.n_qblk - 1 - rest / p.B;
  const int h = kvh * p.g + member;

  const int q0 = qblk * BM;
  const int wq0 = q0 + 32 * wv;
  const int qrow = wq0 + l32;
  const int wq_last = min(wq0 + 31, p.Sq - 1);

  const T* Qb = static_cast<const T*>(p.q) + (int64_t)(b * p.Hq + h) * p.Sq * D;
  const T* Kb = static_cast<const T*>(p.k) + (int64_t)(b * p.Hkv + kvh) * p.Sk * D;
  const T* Vb = static_cast<const T*>(p.v) + (int64_t)(b * p.Hkv + kvh) * p.Sk * D;

  // ---- Q fragment (B operand of S^T): lane holds Q[qrow][hh*HALF, +HALF).
  Frag qf[QF];
  {
    u32x4 qc[HALF / EPC];
    if (qrow < p.Sq) {
      const T* qr = Qb + (int64_t)qrow * D;
      if constexpr (ROPE) {
        const float* cs = p.q_cos + (int64_t)qrow * D;
        const float* sn = p.q_sin + (int64_t)qrow * D;
        const float sgn = hh ? 1.f : -1.f;
#pragma unroll
        for (int c = 0; c < HALF / EPC; ++c) {
          float x[EPC], xp[EPC], y[EPC];
          chunk_to_f32<T>(ldg16(qr + hh * HALF + c * EPC), x);
          chunk_to_f32<T>(ldg16(qr + (1 - hh) * HALF + c * EPC), xp);
#pragma unroll
          for (int e = 0; e < EPC; ++e) {
            const int d = hh * HALF + c * EPC + e;
            y[e] = x[e] * cs[d] + sgn * xp[e] * sn[d];
          }
          qc[c] = f32_to_chunk<T>(y);
        }
      } else {
#pragma unroll
        for (int c = 0; c < HALF / EPC; ++c) qc[c] = ldg16(qr + hh * HALF + c * EPC);
      }
    } else {
#pragma unroll
      for (int c = 0; c < HALF / EPC; ++c) qc[c] = (u32x4){0u, 0u, 0u, 0u};
    }
    // A negative scale is applied as |scale| on -Q (exact sign flips), so the
    // softmax below only ever sees a non-negative scale.
    if (p.scale_log2 < 0.f) {
      const uint32_t sign = ES == 4 ? 0x80000000u : 0x80008000u;
#pragma unroll
      for (int c = 0; c < HALF / EPC; ++c) qc[c] ^= (u32x4){sign, sign, sign, sign};
    }
#pragma unroll
    for (int c = 0; c < HALF / EPC; ++c)
#pragma unroll
      for (int f = 0; f < FPC; ++f) qf[c * FPC + f] = chunk_frag<T>(qc[c], f);
  }

  // ---- staging registers for one K/V block ---------------------------------
  u32x4 kreg[G::K_PER_T][G::K_CHUNKS];
  u32x4 vreg[G::V_PER_T][G::V_CHUNKS];

  // K/V of this (batch, kv head): rows at or past kv_len lie outside the
  // resource and load as zeros (never read from memory).
  const uint32_t kv_bytes = (uint32_t)p.kv_len * (uint32_t)(D * ES);
  const rsrc_t krs = make_rsrc(Kb, kv_bytes);
  const rsrc_t vrs = make_rsrc(Vb, kv_bytes);

  auto load_block = [&](int kv0) {
#pragma unroll
    for (int u = 0; u < G::K_PER_T; ++u) {
      const int c = tid + 256 * u;
      if (G::K_ITEMS % 256 == 0 || c < G::K_ITEMS) {
        const int r = ROPE ? c / (CPR / 2) : c / CPR;
        const int cc = ROPE ? c % (CPR / 2) : c % CPR;
        const uint32_t off = (uint32_t)((kv0 + r) * D + cc * EPC) * ES;
        kreg[u][0] = bufld16(krs, off);
        if constexpr (ROPE) kreg[u][G::K_CHUNKS - 1] = bufld16(krs, off + HALF * ES);
      }
    }
#pragma unroll
    for (int u = 0; u < G::V_PER_T; ++u) {
      const int c = tid + 256 * u;
      if (G::V_ITEMS % 256 == 0 || c < G::V_ITEMS) {
        if constexpr (G::TR) {
          const int r = c / CPR, cc = c % CPR;
          vreg[u][0] = bufld16(vrs, (uint32_t)((kv0 + r) * D + cc * EPC) * ES);
        } else {
          const int kg = c & 15, dc = c >> 4;
#pragma unroll
          for (int r = 0; r < 4; ++r)
            vreg[u][r] = bufld16(vrs, (uint32_t)((kv0 + 4 * kg + r) * D + dc * EPC) * ES);
        }
      }
    }
  };

  auto store_block = [&](int kv0, char* sk, char* sv) {
#pragma unroll
    for (int u = 0; u < G::K_PER_T; ++u) {
      const int c = tid + 256 * u;
      if (G::K_ITEMS % 256 == 0 || c < G::K_ITEMS) {
        if constexpr (ROPE) {
          const int r = c / (CPR / 2), pc = c % (CPR / 2);
          const int key = kv0 + r;
          u32x4 lo_out = {0u, 0u, 0u, 0u}, hi_out = {0u, 0u, 0u, 0u};
          if (key < p.kv_len) {  // tables are [Sk, D]: only read for valid keys
            float lo[EPC], hi[EPC], rlo[EPC], rhi[EPC];
            chunk_to_f32<T>(kreg[u][0], lo);
            chunk_to_f32<T>(kreg[u][1], hi);
            const float* cs = p.k_cos + (int64_t)key * D + pc * EPC;
            const float* sn = p.k_sin + (int64_t)key * D + pc * EPC;
#pragma unroll
            for (int e = 0; e < EPC; ++e) {
              rlo[e] = lo[e] * cs[e] - hi[e] * sn[e];
              rhi[e] = hi[e] * cs[HALF + e] + lo[e] * sn[HALF + e];
            }
            lo_out = f32_to_chunk<T>(rlo);
            hi_out = f32_to_chunk<T>(rhi);
          }
          const int pr = perm_row(r);
          char* dst = sk + pr * (D * ES);
          sts16(dst + 16 * (pc ^ G::kswz(pr)), lo_out);
          sts16(dst + 16 * ((pc + CPR / 2) ^ G::kswz(pr)), hi_out);
        } else {
          const int r = c / CPR, cc = c % CPR;
          const int pr = perm_row(r);
          sts16(sk + pr * (D * ES) + 16 * (cc ^ G::kswz(pr)), kreg[u][0]);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < G::V_PER_T; ++u) {
      const int c = tid + 256 * u;
      if (G::V_ITEMS % 256 == 0 || c < G::V_ITEMS) {
        if constexpr (G::TR) {
          const int r = c / CPR, cc = c % CPR;
          sts16(sv + r * (D * ES) + 16 * (cc ^ G::vswz(r)), vreg[u][0]);
        } else {
          const int kg = c & 15, dc = c >> 4;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const u32x4 o4 = {vreg[u][0][e], vreg[u][1][e], vreg[u][2][e], vreg[u][3][e]};
            sts16(sv + (dc * 4 + e) * G::VT_PITCH + kg * 16, o4);
          }
        }
      }
    }
  };

  float m_run = kNegInf;  // running max, log2 domain (identical in both halves)
  float l_run = 0.f;      // running sum over this lane half's keys
  f32x16 acc[NDT];
#pragma unroll
  for (int i = 0; i < NDT; ++i) acc[i] = (f32x16)(0.f);

  int kv_end = p.kv_len;
  if constexpr (CAUSAL) kv_end = min(kv_end, min(q0 + BM, p.Sq));
  const int nblk = (kv_end + BN - 1) / BN;
  const float c2 = fabsf(p.scale_log2);

  // Per-lane byte offsets of the V^T fragment reads (16-bit types). Lane
  // (group gq = lane/16, j = lane%16) points at V[32(gq/2) + 8c + 4r + j/4]
  // [32dt + 16(gq%2) + 4(j%4)]; the row swizzle only depends on row%4 =
  // (j/4)%4, so the per-dt chunk offsets are lane constants.
  const int tr_g = lane >> 4, tr_j = lane & 15;
  const int tr_row0 = 32 * (tr_g >> 1) + (tr_j >> 2);
  const int tr_col0 = 16 * (tr_g & 1) + 4 * (tr_j & 3);
  const int tr_sw = G::TR ? G::vswz(tr_row0) : 0;
  const int tr_base = tr_row0 * (D * ES) + 16 * (tr_col0 >> 3) + 2 * (tr_col0 & 7);
  int tr_dt[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) tr_dt[dt] = tr_base + 16 * ((4 * dt) ^ tr_sw);

  if (nblk > 0) {
    load_block(0);
    store_block(0, smem, smem + G::K_BYTES);
  }
  __syncthreads();

  for (int j = 0; j < nblk; ++j) {
    const int kv0 = j * BN;
    char* const sk = smem + (j & 1) * (G::K_BYTES + G::V_BYTES);
    char* const sv = sk + G::K_BYTES;
    const bool has_next = j + 1 < nblk;
    if (has_next) load_block(kv0 + BN);

    const bool live = wq0 < p.Sq && !(CAUSAL && kv0 > wq_last);
    if (live) {
      // ---- S^T = K . Q^T --------------------------------------------------
      f32x16 s[2];
      s[0] = (f32x16)(0.f);
      s[1] = (f32x16)(0.f);
      {
        const char* kr0 = sk + l32 * (D * ES);
        const char* kr1 = sk + (32 + l32) * (D * ES);
        const int sw0 = G::kswz(l32), sw1 = G::kswz(32 + l32);
#pragma unroll
        for (int c = 0; c < HALF / EPC; ++c) {
          const int ch = hh * (CPR / 2) + c;
          const u32x4 a0 = lds16(kr0 + 16 * (ch ^ sw0));
          const u32x4 a1 = lds16(kr1 + 16 * (ch ^ sw1));
#pragma unroll
          for (int f = 0; f < FPC; ++f) {
            s[0] = MF::run(chunk_frag<T>(a0, f), qf[c * FPC + f], s[0]);
            s[1] = MF::run(chunk_frag<T>(a1, f), qf[c * FPC + f], s[1]);
          }
        }
      }

      // ---- online softmax (lane owns query qrow; keys kv0 + 32hh + 16t + r)
      // c2 = |scale| * log2(e) >= 0. The running reference m_run only moves
      // when some row's max grows by more than 8 (log2 units): p = 2^(x - m)
      // then stays below 2^8, and since l and acc share the reference the
      // result is unchanged while the O rescale becomes rare.
      const bool need_mask = (kv0 + BN > p.kv_len) || (CAUSAL && kv0 + BN - 1 > wq0);
      float mx = kNegInf;
      if (need_mask) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = kv0 + 32 * hh + 16 * t + r;
            const bool ok = key < p.kv_len && (!CAUSAL || key <= qrow);
            mx = fmaxf(mx, ok ? s[t][r] : kNegInf);
          }
      } else {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[t][r]);
      }
      mx = wave_xor32_max(mx);
      mx = (mx == kNegInf) ? kNegInf : mx * c2;
      const float m_cand = fmaxf(m_run, mx);
      if (__any(m_cand > m_run + 8.f)) {
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_cand);
#pragma unroll
        for (int i = 0; i < NDT; ++i) acc[i] *= alpha;
        l_run *= alpha;
        m_run = m_cand;
      }
      const float m_use = (m_run == kNegInf) ? 0.f : m_run;
      float rs = 0.f;
      if (need_mask) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = kv0 + 32 * hh + 16 * t + r;
            const bool ok = key < p.kv_len && (!CAUSAL || key <= qrow);
            const float e = ok ? __builtin_amdgcn_exp2f(fmaf(s[t][r], c2, -m_use)) : 0.f;
            s[t][r] = e;
            rs += e;
          }
      } else {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float e = __builtin_amdgcn_exp2f(fmaf(s[t][r], c2, -m_use));
            s[t][r] = e;
            rs += e;
          }
      }
      l_run += rs;

      // ---- P fragments (B operand of O^T): keys 32hh + m, m = 0..31 --------
      Frag pfr[PF];
      pack_frags<T>(s[0], s[1], pfr);

      // ---- O^T += V^T . P^T -------------------------------------------------
      if constexpr (G::TR) {
        typedef short v4i16 __attribute__((ext_vector_type(4)));
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            v4i16 part[2];
#pragma unroll
            for (int r = 0; r < 2; ++r) {
              const char* a = sv + tr_dt[dt] + (8 * c + 4 * r) * (D * ES);
              part[r] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                  (__attribute__((address_space(3))) v4i16*)(a));
            }
            const Frag af = __builtin_bit_cast(Frag, __builtin_shufflevector(part[0], part[1], 0, 1, 2, 3, 4, 5, 6, 7));
            acc[dt] = MF::run(af, pfr[c], acc[dt]);
          }
      } else {
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          const char* vr = sv + (32 * dt + l32) * G::VT_PITCH + hh * 32 * ES;
#pragma unroll
          for (int c = 0; c < 32 * ES / 16; ++c) {
            const u32x4 a = lds16(vr + c * 16);
#pragma unroll
            for (int f = 0; f < FPC; ++f) acc[dt] = MF::run(chunk_frag<T>(a, f), pfr[c * FPC + f], acc[dt]);
          }
        }
      }
    }

    if (has_next) {
      char* const nk = smem + ((j + 1) & 1) * (G::K_BYTES + G::V_BYTES);
      store_block(kv0 + BN, nk, nk + G::K_BYTES);
    }
    __syncthreads();
  }

  // ---- finalize: o = acc / l, lse = m ln2 + ln l ---------------------------
  const float l_tot = wave_xor32_sum(l_run);
  if (qrow < p.Sq) {
    const float safe = (l_tot == 0.f) ? 1.f : l_tot;
    T* orow = static_cast<T*>(p.o) + ((int64_t)(b * p.Hq + h) * p.Sq + qrow) * D;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d0 = 32 * dt + 8 * r4 + 4 * hh;
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = acc[dt][4 * r4 + e] / safe;
        if constexpr (ES == 4) {
          *reinterpret_cast<f32x4*>(orow + d0) = (f32x4){y[0], y[1], y[2], y[3]};
        } else {
          typedef T v4 __attribute__((ext_vector_type(4)));
          v4 x;
#pragma unroll
          for (int e = 0; e < 4; ++e) x[e] = Elem<T>::from_f32(y[e]);
          *reinterpret_cast<v4*>(orow + d0) = x;
        }
      }
    if (hh == 0 && p.lse != nullptr) {
      p.lse[(int64_t)(b * p.Hq + h) * p.Sq + qrow] =
          (l_tot == 0.f) ? 0.f : m_run * kLn2 + logf(l_tot);
    }
  }
}

template <typename T, int D>
hipError_t launch_typed(const FwdParams& p, bool causal, bool rope, hipStream_t st) {
  const dim3 grid(p.n_work), block(256);
  if (causal) {
    if (rope) hipLaunchKernelGGL((pf_attn_fwd_kernel<T, D, true, true>), grid, block, 0, st, p);
    else hipLaunchKernelGGL((pf_attn_fwd_kernel<T, D, true, false>), grid, block, 0, st, p);
  } else {
    if (rope) hipLaunchKernelGGL((pf_attn_fwd_kernel<T, D, false, true>), grid, block, 0, st, p);
    else hipLaunchKernelGGL((pf_attn_fwd_kernel<T, D, false, false>), grid, block, 0, st, p);
  }
  return hipGetLastError();
}

template <typename T>
hipError_t launch_dim(const FwdParams& p, int head_dim, bool causal, bool rope, hipStream_t st) {
  if (head_dim == 128) return launch_typed<T, 128>(p, causal, rope, st);
  if (head_dim == 64) return launch_typed<T, 64>(p, causal, rope, st);
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_attn_fwd(const FwdParams& p, int dtype, int head_dim, bool causal, bool rope,
                           hipStream_t stream) {
  switch (dtype) {
    case kF32: return launch_dim<float>(p, head_dim, causal, rope, stream);
    case kBF16: return launch_dim<bf16_t>(p, head_dim, causal, rope, stream);
    case kF16: return launch_dim<f16_t>(p, head_dim, causal, rope, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace pf
