// Forward prefill attention for gfx950 (CDNA4), with optional fused RoPE.
//
// Replaces the reference's `flash_attention_fwd` pallas_call
// (flash_attention.py:162-227, kernel :61-159) and `flash_attention_rope_fwd`
// (fused_rope.py:183-213, kernel :53-113).
//
// Work decomposition: one workgroup of 4 waves per (batch, query head, 128-row
// query block); each wave owns 32 query rows. The grid is 1-D: heavy (late)
// query blocks first for causal load balance, and the query heads of one GQA
// group on one XCD so they hit the same L2 for K/V (see xcd_remap).
//
// Per 64-key block: K [64 x D] is staged in LDS row-major; V is staged
// transposed (V^T [D x 64]) because P.V contracts over keys and an MFMA
// operand must hold its reduction index contiguously per lane.
//   S^T = K . Q^T   (A = K rows from LDS, B = Q held in registers)
//   O^T += V^T . P^T (A = V^T rows from LDS, B = P from the S^T accumulators)
// With S^T, lane l owns query l%32: the online-softmax row statistics are
// in-lane except one exchange between the two lane halves. K rows are stored
// in LDS in a permuted order so that lane half hh's 32 accumulator values
// are keys [32hh, 32hh+32) of the block in order, exactly the k-slots the
// P^T operand needs -- no cross-lane shuffle of P.
//
// Semantics (flash_attention.py): mask k >= kv_len and (causal) k > q, with
// K/V rows past kv_len never read (zero-filled) (:95-120); online softmax in
// float32 (:123-134); whole-tile skipping (:136-147); o = acc / l with l == 0
// giving o = 0 and lse = 0 (:150-159); lse is the natural log-sum-exp of the
// scaled scores. Scores are kept in the log2 domain (exp2 with log2(e) folded
// into the scale) and converted back for the LSE.
#include "pf_common.hpp"
#include "pf_kernels.hpp"

namespace pf {

namespace {

constexpr int kFwdBM = 128;  // query rows per workgroup
constexpr int kFwdBN = 64;   // keys per block

// LDS row of key r (0..63) inside a staged K block: MFMA tile t = (r>>4)&1 row
// 8*((r>>2)&3) + 4*(r>>5) + (r&3). Lane half hh then reads back keys
// 32hh + 16t + reg for accumulator register `reg`.
__device__ inline int k_lds_row(int r) {
  return ((r >> 4) & 1) * 32 + ((r >> 2) & 3) * 8 + (r >> 5) * 4 + (r & 3);
}

template <typename T, int D, bool CAUSAL, bool ROPE>
__global__ __launch_bounds__(256, 2) void pf_attn_fwd_kernel(FwdParams p) {
  using MF = Mfma32<T>;
  using Frag = typename MF::Frag;
  constexpr int BM = kFwdBM, BN = kFwdBN;
  constexpr int HALF = D / 2;
  constexpr int ES = sizeof(T);
  constexpr int EPC = 16 / ES;   // elements per 16-byte chunk
  constexpr int CPR = D / EPC;   // chunks per row
  constexpr int KP = D * ES + 16;   // K tile row pitch (bytes)
  constexpr int VP = BN * ES + 16;  // V^T tile row pitch (bytes)
  constexpr int FPC = frags_per_chunk<T>();
  constexpr int QF = HALF / MF::kK;  // Q fragments per lane
  constexpr int NDT = D / 32;        // 32-row tiles of O^T
  constexpr int PF = 32 / MF::kK;    // P fragments per lane per block
  static_assert(BM == 128 && BN == 64, "tile shape is baked into the lane maps");

  __shared__ __attribute__((aligned(16))) char smem[BN * KP + D * VP];
  char* const sk = smem;
  char* const sv = smem + BN * KP;

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
#pragma unroll
    for (int c = 0; c < HALF / EPC; ++c)
#pragma unroll
      for (int f = 0; f < FPC; ++f) qf[c * FPC + f] = chunk_frag<T>(qc[c], f);
  }

  float m_run = kNegInf;  // running max, log2 domain (identical in both halves)
  float l_run = 0.f;      // running sum over this lane half's keys
  f32x16 acc[NDT];
#pragma unroll
  for (int i = 0; i < NDT; ++i) acc[i] = (f32x16)(0.f);

  int kv_end = p.kv_len;
  if constexpr (CAUSAL) kv_end = min(kv_end, min(q0 + BM, p.Sq));
  const int nblk = (kv_end + BN - 1) / BN;

  for (int j = 0; j < nblk; ++j) {
    const int kv0 = j * BN;
    __syncthreads();  // previous block's LDS reads are done

    // ---- stage K (row-permuted) -------------------------------------------
    if constexpr (!ROPE) {
#pragma unroll
      for (int u = 0; u < BN * CPR / 256; ++u) {
        const int c = tid + 256 * u;
        const int r = c / CPR, cc = c % CPR;
        const int key = kv0 + r;
        const u32x4 val = (key < p.kv_len) ? ldg16(Kb + (int64_t)key * D + cc * EPC)
                                           : (u32x4){0u, 0u, 0u, 0u};
        sts16(sk + k_lds_row(r) * KP + cc * 16, val);
      }
    } else {
      constexpr int HC = CPR / 2;  // chunks per half row
#pragma unroll
      for (int u = 0; u < (BN * HC + 255) / 256; ++u) {
        const int c = tid + 256 * u;
        if (BN * HC % 256 == 0 || c < BN * HC) {
          const int r = c / HC, pc = c % HC;
          const int key = kv0 + r;
          u32x4 lo_out = {0u, 0u, 0u, 0u}, hi_out = {0u, 0u, 0u, 0u};
          if (key < p.kv_len) {
            float lo[EPC], hi[EPC], rlo[EPC], rhi[EPC];
            chunk_to_f32<T>(ldg16(Kb + (int64_t)key * D + pc * EPC), lo);
            chunk_to_f32<T>(ldg16(Kb + (int64_t)key * D + HALF + pc * EPC), hi);
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
          char* dst = sk + k_lds_row(r) * KP;
          sts16(dst + pc * 16, lo_out);
          sts16(dst + (pc + HC) * 16, hi_out);
        }
      }
    }

    // ---- stage V transposed: V^T[d][key] ----------------------------------
    {
      constexpr int NDC = D / EPC;
#pragma unroll
      for (int u = 0; u < (16 * NDC + 255) / 256; ++u) {
        const int c = tid + 256 * u;
        if (16 * NDC % 256 == 0 || c < 16 * NDC) {
          const int kg = c & 15, dc = c >> 4;
          u32x4 ch[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int key = kv0 + 4 * kg + r;
            ch[r] = (key < p.kv_len) ? ldg16(Vb + (int64_t)key * D + dc * EPC)
                                     : (u32x4){0u, 0u, 0u, 0u};
          }
          if constexpr (ES == 4) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const u32x4 o4 = {ch[0][e], ch[1][e], ch[2][e], ch[3][e]};
              sts16(sv + (dc * 4 + e) * VP + kg * 16, o4);
            }
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const int wd = e >> 1, sh = (e & 1) * 16;
              const uint32_t v0 = (ch[0][wd] >> sh) & 0xffffu, v1 = (ch[1][wd] >> sh) & 0xffffu;
              const uint32_t v2 = (ch[2][wd] >> sh) & 0xffffu, v3 = (ch[3][wd] >> sh) & 0xffffu;
              const u32x2 o2 = {v0 | (v1 << 16), v2 | (v3 << 16)};
              *reinterpret_cast<u32x2*>(sv + (dc * 8 + e) * VP + kg * 8) = o2;
            }
          }
        }
      }
    }
    __syncthreads();

    if (wq0 >= p.Sq) continue;                // wave has no query rows
    if (CAUSAL && kv0 > wq_last) continue;    // block entirely in this wave's future

    // ---- S^T = K . Q^T ----------------------------------------------------
    f32x16 s[2];
    s[0] = (f32x16)(0.f);
    s[1] = (f32x16)(0.f);
    {
      const char* kr0 = sk + l32 * KP + hh * HALF * ES;
      const char* kr1 = sk + (32 + l32) * KP + hh * HALF * ES;
#pragma unroll
      for (int c = 0; c < HALF / EPC; ++c) {
        const u32x4 a0 = lds16(kr0 + c * 16);
        const u32x4 a1 = lds16(kr1 + c * 16);
#pragma unroll
        for (int f = 0; f < FPC; ++f) {
          s[0] = MF::run(chunk_frag<T>(a0, f), qf[c * FPC + f], s[0]);
          s[1] = MF::run(chunk_frag<T>(a1, f), qf[c * FPC + f], s[1]);
        }
      }
    }

    // ---- online softmax (lane owns query qrow; keys kv0 + 32hh + 16t + r) --
    const bool need_mask = (kv0 + BN > p.kv_len) || (CAUSAL && kv0 + BN - 1 > wq0);
    float mx = kNegInf;
    if (need_mask) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kv0 + 32 * hh + 16 * t + r;
          const bool ok = key < p.kv_len && (!CAUSAL || key <= qrow);
          const float x = ok ? s[t][r] * p.scale_log2 : kNegInf;
          s[t][r] = x;
          mx = fmaxf(mx, x);
        }
    } else {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float x = s[t][r] * p.scale_log2;
          s[t][r] = x;
          mx = fmaxf(mx, x);
        }
    }
    mx = wave_xor32_max(mx);
    const float m_new = fmaxf(m_run, mx);
    const float m_use = (m_new == kNegInf) ? 0.f : m_new;
    const float alpha = exp2f(m_run - m_use);
    float rs = 0.f;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float e = exp2f(s[t][r] - m_use);
        s[t][r] = e;
        rs += e;
      }
    l_run = l_run * alpha + rs;
    m_run = m_new;
#pragma unroll
    for (int i = 0; i < NDT; ++i) acc[i] *= alpha;

    // ---- P fragments (B operand of O^T): keys 32hh + m, m = 0..31 ----------
    Frag pfr[PF];
    if constexpr (ES == 4) {
#pragma unroll
      for (int m = 0; m < 32; ++m) pfr[m] = s[m >> 4][m & 15];
    } else {
#pragma unroll
      for (int f = 0; f < PF; ++f) {
        Frag x;
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = Elem<T>::from_f32(s[f >> 1][8 * (f & 1) + e]);
        pfr[f] = x;
      }
    }

    // ---- O^T += V^T . P^T ---------------------------------------------------
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const char* vr = sv + (32 * dt + l32) * VP + hh * 32 * ES;
#pragma unroll
      for (int c = 0; c < 32 * ES / 16; ++c) {
        const u32x4 a = lds16(vr + c * 16);
#pragma unroll
        for (int f = 0; f < FPC; ++f) acc[dt] = MF::run(chunk_frag<T>(a, f), pfr[c * FPC + f], acc[dt]);
      }
    }
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
