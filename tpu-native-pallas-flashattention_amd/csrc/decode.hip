// Single-query decode attention for gfx950: contiguous KV cache and paged pool.
//
// Replaces `flash_attention_decode` (flash_attention.py:555-589: the forward
// pallas_call with block_q = 1, kv_len = cache_len) and the
// `paged_flash_attention` pallas_call (paged.py:151-192, kernel :45-99).
//
// Design (bandwidth-bound, arithmetic intensity ~4 FLOP/B):
//  * Split-KV: one wave per (batch, kv head, 32-head slice of the GQA group,
//    key chunk). All query heads of a group ride in one wave as the N columns
//    of the MFMA, so every K/V byte is read from HBM exactly once (the
//    reference grid runs per query head and re-streams each KV head g times).
//  * S^T = K . Q^T on 32x32 MFMA with K read straight from global memory as
//    the A operand (lane = key row, 16-byte loads of a contiguous d range).
//  * V is staged transposed through a wave-private LDS slice (P.V contracts
//    over keys), then O^T += V^T . P^T on MFMA. Waves never wait on each
//    other: each owns its LDS slice and synchronises only with itself.
//  * Partial (max, sum, unnormalised acc) per chunk go to the workspace; a
//    combine kernel merges them with log-sum-exp algebra and casts.
// Masking: keys at or past the valid length are never read (their K/V rows
// are zero-filled), so a NaN tail or -1 table padding cannot leak
// (flash_attention.py:95-100; paged.py:73-80, :93). Paged: table entries are
// read only for logical pages below ceil(len / page_size) and clamped into
// [0, num_pages).
#include "pf_common.hpp"
#include "pf_kernels.hpp"

namespace pf {

namespace {

constexpr int kDecBN = 64;  // keys per block

// Wave-scope ordering of this wave's own LDS traffic: LDS operations of one
// wavefront execute in order, so only compiler reordering must be prevented.
__device__ inline void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Row `key` of (b, kv head) in the cache or pool; rows are p.dr elements.
template <typename T, bool PAGED>
__device__ inline const T* key_row(const DecodeParams& p, const T* base, int b, int kvh, int key) {
  if constexpr (PAGED) {
    const int lp = key / p.page_size;
    int page = p.block_tables[(int64_t)b * p.pages_per_seq + lp];
    page = min(max(page, 0), p.num_pages - 1);
    const int off = key - lp * p.page_size;
    return base + (((int64_t)page * p.Hkv + kvh) * p.page_size + off) * p.dr;
  } else {
    return base + ((int64_t)(b * p.Hkv + kvh) * p.cache_size + key) * p.dr;
  }
}

template <typename T, int D, bool PAGED>
__global__ __launch_bounds__(256, (kWgPerCu<T, D>)) void pf_decode_kernel(DecodeParams p) {
  using MF = Mfma32<T>;
  using Frag = typename MF::Frag;
  constexpr int BN = kDecBN;
  constexpr int HALF = D / 2;
  constexpr int ES = sizeof(T);
  constexpr int EPC = 16 / ES;
  constexpr int VP = BN * ES + 16;  // V^T row pitch (bytes)
  constexpr int FPC = frags_per_chunk<T>();
  constexpr int QF = HALF / MF::kK;
  constexpr int NDT = D / 32;
  constexpr int PF = 32 / MF::kK;
  constexpr int NDC = D / EPC;       // 16-byte chunks per row

  __shared__ __attribute__((aligned(16))) char smem[4 * D * VP];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int hh = lane >> 5;
  const int l32 = lane & 31;
  char* const sv = smem + wv * D * VP;

  const int g = p.Hq / p.Hkv;
  const int n_hc = (g + 31) / 32;
  const int task = blockIdx.x * 4 + wv;
  const int n_tasks = p.B * p.Hkv * n_hc * p.n_split;
  if (task >= n_tasks) return;  // wave-private work: no workgroup barrier below
  const int split = task % p.n_split;
  int rest = task / p.n_split;
  const int hc = rest % n_hc;
  rest /= n_hc;
  const int kvh = rest % p.Hkv;
  const int b = rest / p.Hkv;

  int L;
  if constexpr (PAGED) {
    L = min(max(p.context_lens[b], 0), p.pages_per_seq * p.page_size);
  } else {
    L = p.cache_len;
  }
  const int k_begin = split * p.chunk;
  if (k_begin >= L) return;  // empty chunk: the combine never reads it
  const int k_end = min(L, k_begin + p.chunk);

  const int qh = hc * 32 + l32;  // query head inside the group
  const bool qvalid = qh < g;
  const int h = kvh * g + (qvalid ? qh : 0);

  const T* Kbase = static_cast<const T*>(p.k);
  const T* Vbase = static_cast<const T*>(p.v);

  // Stored head dim: columns [dr, D) are zeros (never read).
  const int dr = p.dr;
  auto col_ok = [&](int col) { return col < dr; };  // col: first column of a 16-byte chunk

  // Q fragment (B operand): lane holds Q[b, h, 0, hh*HALF .. +HALF)
  Frag qf[QF];
  {
    const T* qr = static_cast<const T*>(p.q) + (int64_t)(b * p.Hq + h) * dr + hh * HALF;
#pragma unroll
    for (int c = 0; c < HALF / EPC; ++c) {
      const u32x4 ch = (qvalid && col_ok(hh * HALF + c * EPC)) ? ldg16(qr + c * EPC) : (u32x4){0u, 0u, 0u, 0u};
#pragma unroll
      for (int f = 0; f < FPC; ++f) qf[c * FPC + f] = chunk_frag<T>(ch, f);
    }
  }

  float m_run = kNegInf, l_run = 0.f;
  f32x16 acc[NDT];
#pragma unroll
  for (int i = 0; i < NDT; ++i) acc[i] = (f32x16)(0.f);

  for (int kv0 = k_begin; kv0 < k_end; kv0 += BN) {
    // ---- K fragments straight from global: tile t, row R = l32 holds key
    //      kv0 + 32*((R>>2)&1) + 16t + 4*(R>>3) + (R&3)
    u32x4 kc[2][HALF / EPC];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int key = kv0 + 32 * ((l32 >> 2) & 1) + 16 * t + 4 * (l32 >> 3) + (l32 & 3);
      if (key < k_end) {
        const T* kr = key_row<T, PAGED>(p, Kbase, b, kvh, key) + hh * HALF;
#pragma unroll
        for (int c = 0; c < HALF / EPC; ++c)
          kc[t][c] = col_ok(hh * HALF + c * EPC) ? ldg16(kr + c * EPC) : (u32x4){0u, 0u, 0u, 0u};
      } else {
#pragma unroll
        for (int c = 0; c < HALF / EPC; ++c) kc[t][c] = (u32x4){0u, 0u, 0u, 0u};
      }
    }

    // ---- V rows -> registers (4 keys x 16 bytes per item) -------------------
    constexpr int NITEM = (16 * NDC + 63) / 64;
    u32x4 vc[NITEM][4];
#pragma unroll
    for (int u = 0; u < NITEM; ++u) {
      const int c = lane + 64 * u;
      const int kg = c & 15, dc = c >> 4;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kv0 + 4 * kg + r;
        if ((16 * NDC % 64 == 0 || c < 16 * NDC) && key < k_end && col_ok(dc * EPC))
          vc[u][r] = ldg16(key_row<T, PAGED>(p, Vbase, b, kvh, key) + dc * EPC);
        else
          vc[u][r] = (u32x4){0u, 0u, 0u, 0u};
      }
    }

    // ---- S^T = K . Q^T ----------------------------------------------------
    f32x16 s[2];
    s[0] = (f32x16)(0.f);
    s[1] = (f32x16)(0.f);
#pragma unroll
    for (int c = 0; c < HALF / EPC; ++c)
#pragma unroll
      for (int f = 0; f < FPC; ++f) {
        s[0] = MF::run(chunk_frag<T>(kc[0][c], f), qf[c * FPC + f], s[0]);
        s[1] = MF::run(chunk_frag<T>(kc[1][c], f), qf[c * FPC + f], s[1]);
      }

    // ---- V^T into this wave's LDS slice -----------------------------------
    wave_lds_sync();  // previous block's V^T reads are done
#pragma unroll
    for (int u = 0; u < NITEM; ++u) {
      const int c = lane + 64 * u;
      if (16 * NDC % 64 == 0 || c < 16 * NDC) {
        const int kg = c & 15, dc = c >> 4;
        if constexpr (ES == 4) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const u32x4 o4 = {vc[u][0][e], vc[u][1][e], vc[u][2][e], vc[u][3][e]};
            sts16(sv + (dc * 4 + e) * VP + kg * 16, o4);
          }
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int wd = e >> 1, sh = (e & 1) * 16;
            const uint32_t v0 = (vc[u][0][wd] >> sh) & 0xffffu, v1 = (vc[u][1][wd] >> sh) & 0xffffu;
            const uint32_t v2 = (vc[u][2][wd] >> sh) & 0xffffu, v3 = (vc[u][3][wd] >> sh) & 0xffffu;
            const u32x2 o2 = {v0 | (v1 << 16), v2 | (v3 << 16)};
            *reinterpret_cast<u32x2*>(sv + (dc * 8 + e) * VP + kg * 8) = o2;
          }
        }
      }
    }
    wave_lds_sync();

    // ---- online softmax over keys kv0 + 32hh + 16t + r ---------------------
    float mx = kNegInf;
    const bool need_mask = kv0 + BN > k_end;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kv0 + 32 * hh + 16 * t + r;
        const float x = (!need_mask || key < k_end) ? s[t][r] * p.scale_log2 : kNegInf;
        s[t][r] = x;
        mx = fmaxf(mx, x);
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

  // ---- partial (m, l, acc) for this chunk ---------------------------------
  const float l_tot = wave_xor32_sum(l_run);
  if (qvalid) {
    const int64_t slot = (int64_t)(b * p.Hq + h) * p.n_split + split;
    float* po = p.part_o + slot * D;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d0 = 32 * dt + 8 * r4 + 4 * hh;
        *reinterpret_cast<f32x4*>(po + d0) =
            (f32x4){acc[dt][4 * r4], acc[dt][4 * r4 + 1], acc[dt][4 * r4 + 2], acc[dt][4 * r4 + 3]};
      }
    if (hh == 0) {
      p.part_ml[slot * 2 + 0] = m_run;
      p.part_ml[slot * 2 + 1] = l_tot;
    }
  }
}

// Merge the per-chunk partials of one (b, h): o = sum_s acc_s 2^(m_s - M) /
// sum_s l_s 2^(m_s - M); an empty row (no valid key) gives o = 0
// (flash_attention.py:150-159; paged.py:95-99).
template <typename T, int D, bool PAGED>
__global__ __launch_bounds__(256) void pf_decode_combine_kernel(DecodeParams p) {
  const int lane = threadIdx.x & 63;
  const int bh = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (bh >= p.B * p.Hq) return;
  const int b = bh / p.Hq;
  int L;
  if constexpr (PAGED) {
    L = min(max(p.context_lens[b], 0), p.pages_per_seq * p.page_size);
  } else {
    L = p.cache_len;
  }
  const int n_valid = (L + p.chunk - 1) / p.chunk;
  const float* ml = p.part_ml + (int64_t)bh * p.n_split * 2;
  const float* po = p.part_o + (int64_t)bh * p.n_split * D;
  float M = kNegInf;
  for (int s = 0; s < n_valid; ++s) M = fmaxf(M, ml[2 * s]);
  const float Mu = (M == kNegInf) ? 0.f : M;
  constexpr int PER = D / 64;
  float o[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) o[e] = 0.f;
  float lsum = 0.f;
  for (int s = 0; s < n_valid; ++s) {
    const float w = exp2f(ml[2 * s] - Mu);
    lsum += ml[2 * s + 1] * w;
#pragma unroll
    for (int e = 0; e < PER; ++e) o[e] += po[(int64_t)s * D + lane * PER + e] * w;
  }
  const float safe = (lsum == 0.f) ? 1.f : lsum;
  T* out = static_cast<T*>(p.o) + (int64_t)bh * p.dr;
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    const int col = lane * PER + e;
    if (col < p.dr) out[col] = Elem<T>::from_f32(o[e] / safe);
  }
}

template <typename T, int D, bool PAGED>
hipError_t launch_typed(const DecodeParams& p, hipStream_t st) {
  const int g = p.Hq / p.Hkv;
  const int n_hc = (g + 31) / 32;
  const int64_t n_tasks = (int64_t)p.B * p.Hkv * n_hc * p.n_split;
  hipLaunchKernelGGL((pf_decode_kernel<T, D, PAGED>), dim3((unsigned)((n_tasks + 3) / 4)), dim3(256),
                     0, st, p);
  return hipGetLastError();
}

template <typename T, int D, bool PAGED>
hipError_t launch_combine_typed(const DecodeParams& p, hipStream_t st) {
  const int64_t n_bh = (int64_t)p.B * p.Hq;
  hipLaunchKernelGGL((pf_decode_combine_kernel<T, D, PAGED>), dim3((unsigned)((n_bh + 3) / 4)),
                     dim3(256), 0, st, p);
  return hipGetLastError();
}

template <typename T, bool PAGED>
hipError_t launch_dim(const DecodeParams& p, bool combine, hipStream_t st) {
  if (p.D == 128) return combine ? launch_combine_typed<T, 128, PAGED>(p, st) : launch_typed<T, 128, PAGED>(p, st);
  if (p.D == 64) return combine ? launch_combine_typed<T, 64, PAGED>(p, st) : launch_typed<T, 64, PAGED>(p, st);
  if constexpr (sizeof(T) == 2)
    if (p.D == 256)
      return combine ? launch_combine_typed<T, 256, PAGED>(p, st) : launch_typed<T, 256, PAGED>(p, st);
  return hipErrorInvalidValue;
}

template <bool PAGED>
hipError_t launch_dtype(const DecodeParams& p, int dtype, bool combine, hipStream_t st) {
  switch (dtype) {
    case kF32: return launch_dim<float, PAGED>(p, combine, st);
    case kBF16: return launch_dim<bf16_t, PAGED>(p, combine, st);
    case kF16: return launch_dim<f16_t, PAGED>(p, combine, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_decode_combine(const DecodeParams& p, int dtype, bool paged, hipStream_t stream) {
  return paged ? launch_dtype<true>(p, dtype, true, stream) : launch_dtype<false>(p, dtype, true, stream);
}

hipError_t launch_decode(const DecodeParams& p, int dtype, bool paged, hipStream_t stream) {
  // the streaming kernel reads rows of exactly its compute width
  if (p.dr == p.D && decode_stream_supported(dtype, p.dr, paged, p.page_size))
    return launch_decode_stream(p, dtype, paged, stream);
  hipError_t e = paged ? launch_dtype<true>(p, dtype, false, stream) : launch_dtype<false>(p, dtype, false, stream);
  if (e != hipSuccess) return e;
  return launch_decode_combine(p, dtype, paged, stream);
}

}  // namespace pf
