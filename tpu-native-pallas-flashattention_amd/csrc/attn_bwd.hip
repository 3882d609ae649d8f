// Backward attention for gfx950: delta preprocess, dQ kernel, dK/dV kernel.
//
// Replaces `_flash_attention_bwd_call` (flash_attention.py:354-442):
//   delta_i = sum_d o_id * do_id            (XLA op, :363-365) -> delta kernel
//   flash_attention_bwd_dq  pallas_call     (:379-398, kernel :276-311)
//   flash_attention_bwd_dkv pallas_call     (:403-431, kernel :314-351)
//   GQA group sum of per-head dK/dV         (:433-436)
// Both gradient kernels recompute p = exp(s - lse) from the forward LSE
// (_bwd_common, :245-273) and apply the same masks: k < kv_len, q < Sq and
// (causal) q >= k. The dK/dV kernel loops over the query heads of its GQA
// group and accumulates dK/dV in registers, so the group sum happens in
// float32 inside the kernel with one cast at the end -- the reference's
// per-head float32 [B, Hq, Sk, D] temporaries and the separate sum pass do
// not exist here.
//
// Layouts (all 32x32 MFMA, float32 accumulation):
//  dQ kernel (workgroup = 128 query rows, 4 waves x 32 rows; loop over 64-key
//  blocks): S^T = K Q^T, dP^T = V dO^T (K, V natural in LDS; Q, dO in
//  registers); dS^T = P^T (dP^T - delta); dQ^T += K^T dS^T (K^T in LDS).
//  dK/dV kernel (workgroup = 128 keys, 4 waves x 32 keys; loop over group
//  heads x 64-row query blocks): S = Q K^T, dP = dO V^T (Q, dO natural in
//  LDS; K, V in registers); dS = P (dP - delta); dV^T += dO^T P,
//  dK^T += Q^T dS (Q^T, dO^T transposed in LDS).
#include "pf_common.hpp"
#include "pf_kernels.hpp"
#include "pf_tiles.hpp"

namespace pf {

namespace {

// ---------------------------------------------------------------------------
// delta[b, h, i] = sum_d f32(o[b,h,i,d]) * f32(do[b,h,i,d])
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(256) void pf_attn_bwd_delta_kernel(BwdParams p) {
  constexpr int EPC = 16 / (int)sizeof(T);
  constexpr int LPR = D / EPC;       // lanes per row
  constexpr int RPB = 256 / LPR;     // rows per workgroup
  const int64_t rows = (int64_t)p.B * p.Hq * p.Sq;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / LPR;
  const int sub = threadIdx.x % LPR;
  float acc = 0.f;
  if (row < rows) {
    float a[EPC], c[EPC];
    chunk_to_f32<T>(ldg16(static_cast<const T*>(p.o) + row * D + sub * EPC), a);
    chunk_to_f32<T>(ldg16(static_cast<const T*>(p.dout) + row * D + sub * EPC), c);
#pragma unroll
    for (int e = 0; e < EPC; ++e) acc += a[e] * c[e];
  }
#pragma unroll
  for (int off = LPR / 2; off >= 1; off >>= 1) acc += __shfl_xor(acc, off);
  if (row < rows && sub == 0) p.delta[row] = acc;
}

// ---------------------------------------------------------------------------
// dQ
// ---------------------------------------------------------------------------
template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void pf_attn_bwd_dq_kernel(BwdParams p, int n_qblk, int n_work) {
  using MF = Mfma32<T>;
  using Frag = typename MF::Frag;
  using G = TileGeom<T, D>;
  constexpr int BM = 128, BN = 64;
  constexpr int QF = (D / 2) / MF::kK;
  constexpr int NDT = D / 32;
  constexpr int PF = 32 / MF::kK;

  __shared__ __attribute__((aligned(16))) char smem[2 * G::NAT_BYTES + G::TRN_BYTES];
  char* const sk = smem;
  char* const sv = smem + G::NAT_BYTES;
  char* const skt = smem + 2 * G::NAT_BYTES;

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, hh = lane >> 5, l32 = lane & 31;
  const int w = xcd_remap(blockIdx.x, n_work, p.g);
  const int member = w % p.g;
  int rest = w / p.g;
  const int kvh = rest % p.Hkv;
  rest /= p.Hkv;
  const int b = rest % p.B;
  const int qblk = n_qblk - 1 - rest / p.B;
  const int h = kvh * p.g + member;

  const int q0 = qblk * BM;
  const int wq0 = q0 + 32 * wv;
  const int qrow = wq0 + l32;
  const bool qvalid = qrow < p.Sq;
  const int wq_last = min(wq0 + 31, p.Sq - 1);

  const int64_t qoff = (int64_t)(b * p.Hq + h) * p.Sq;
  const T* Qb = static_cast<const T*>(p.q) + qoff * D;
  const T* dOb = static_cast<const T*>(p.dout) + qoff * D;
  const T* Kb = static_cast<const T*>(p.k) + (int64_t)(b * p.Hkv + kvh) * p.Sk * D;
  const T* Vb = static_cast<const T*>(p.v) + (int64_t)(b * p.Hkv + kvh) * p.Sk * D;

  Frag qf[QF], dof[QF];
  load_row_frags<T, D>(Qb, qrow, qvalid, hh, qf);
  load_row_frags<T, D>(dOb, qrow, qvalid, hh, dof);
  const float lse2 = qvalid ? p.lse[qoff + qrow] * kLog2e : 0.f;
  const float dlt = qvalid ? p.delta[qoff + qrow] : 0.f;

  f32x16 acc[NDT];
#pragma unroll
  for (int i = 0; i < NDT; ++i) acc[i] = (f32x16)(0.f);

  int kv_end = p.kv_len;
  if constexpr (CAUSAL) kv_end = min(kv_end, min(q0 + BM, p.Sq));
  const int nblk = (kv_end + BN - 1) / BN;

  for (int j = 0; j < nblk; ++j) {
    const int kv0 = j * BN;
    __syncthreads();
    stage_tile<T, D>(Kb, kv0, p.kv_len, sk, skt, tid);
    stage_tile<T, D>(Vb, kv0, p.kv_len, sv, nullptr, tid);
    __syncthreads();
    if (wq0 >= p.Sq) continue;
    if (CAUSAL && kv0 > wq_last) continue;

    f32x16 s0 = (f32x16)(0.f), s1 = (f32x16)(0.f), d0 = (f32x16)(0.f), d1 = (f32x16)(0.f);
    mfma_rows_x_frags<T, D>(sk, l32, hh, qf, s0, s1);
    mfma_rows_x_frags<T, D>(sv, l32, hh, dof, d0, d1);

    // keys kv0 + 32hh + 16t + r, query qrow
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kv0 + 32 * hh + 16 * t + r;
        const bool ok = qvalid && key < p.kv_len && (!CAUSAL || key <= qrow);
        const float sx = t ? s1[r] : s0[r];
        const float dp = t ? d1[r] : d0[r];
        const float pv = ok ? exp2f(sx * p.scale_log2 - lse2) : 0.f;
        const float ds = pv * (dp - dlt);
        if (t) s1[r] = ds; else s0[r] = ds;
      }
    Frag dsf[PF];
    pack_frags<T>(s0, s1, dsf);
    mfma_trn_x_frags<T, D>(skt, l32, hh, dsf, acc);
  }

  if (qvalid) store_acc_row<T, D>(static_cast<T*>(p.dq) + (qoff + qrow) * D, acc, p.sm_scale, hh);
}

// ---------------------------------------------------------------------------
// dK / dV (group-summed)
// ---------------------------------------------------------------------------
template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void pf_attn_bwd_dkv_kernel(BwdParams p, int n_kblk) {
  using MF = Mfma32<T>;
  using Frag = typename MF::Frag;
  using G = TileGeom<T, D>;
  constexpr int BNK = 128, BMQ = 64;
  constexpr int KF = (D / 2) / MF::kK;
  constexpr int NDT = D / 32;
  constexpr int PF = 32 / MF::kK;

  __shared__ __attribute__((aligned(16))) char smem[2 * G::NAT_BYTES + 2 * G::TRN_BYTES + 2 * BMQ * 4];
  char* const sq = smem;
  char* const sdo = smem + G::NAT_BYTES;
  char* const sqt = smem + 2 * G::NAT_BYTES;
  char* const sdot = smem + 2 * G::NAT_BYTES + G::TRN_BYTES;
  float* const slse = reinterpret_cast<float*>(smem + 2 * G::NAT_BYTES + 2 * G::TRN_BYTES);
  float* const sdl = slse + BMQ;

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, hh = lane >> 5, l32 = lane & 31;
  // heavy first: for causal, early key blocks are attended by the most queries
  const int w = blockIdx.x;
  const int kblk = w / (p.B * p.Hkv);
  const int bk = w % (p.B * p.Hkv);
  const int b = bk / p.Hkv, kvh = bk % p.Hkv;

  const int k0 = kblk * BNK;
  const int wk0 = k0 + 32 * wv;
  const int kkey = wk0 + l32;
  const bool kvalid = kkey < p.kv_len;

  const int64_t koff = (int64_t)(b * p.Hkv + kvh) * p.Sk;
  Frag kf[KF], vf[KF];
  load_row_frags<T, D>(static_cast<const T*>(p.k) + koff * D, kkey, kvalid, hh, kf);
  load_row_frags<T, D>(static_cast<const T*>(p.v) + koff * D, kkey, kvalid, hh, vf);

  f32x16 dk[NDT], dv[NDT];
#pragma unroll
  for (int i = 0; i < NDT; ++i) {
    dk[i] = (f32x16)(0.f);
    dv[i] = (f32x16)(0.f);
  }

  const bool wave_live = wk0 < p.kv_len;
  const int q_begin = CAUSAL ? (k0 / BMQ) * BMQ : 0;
  // keys of the whole workgroup at or past kv_len: gradients are exactly zero
  const int n_members = (k0 < p.kv_len) ? p.g : 0;

  for (int member = 0; member < n_members; ++member) {
    const int h = kvh * p.g + member;
    const int64_t qoff = (int64_t)(b * p.Hq + h) * p.Sq;
    const T* Qb = static_cast<const T*>(p.q) + qoff * D;
    const T* dOb = static_cast<const T*>(p.dout) + qoff * D;
    for (int qb0 = q_begin; qb0 < p.Sq; qb0 += BMQ) {
      __syncthreads();
      stage_tile<T, D>(Qb, qb0, p.Sq, sq, sqt, tid);
      stage_tile<T, D>(dOb, qb0, p.Sq, sdo, sdot, tid);
      if (tid < BMQ) {
        const int q = qb0 + tid;
        slse[tid] = q < p.Sq ? p.lse[qoff + q] * kLog2e : 0.f;
        sdl[tid] = q < p.Sq ? p.delta[qoff + q] : 0.f;
      }
      __syncthreads();
      if (!wave_live) continue;
      if (CAUSAL && qb0 + BMQ - 1 < wk0) continue;  // all these queries precede the wave's keys

      f32x16 s0 = (f32x16)(0.f), s1 = (f32x16)(0.f), d0 = (f32x16)(0.f), d1 = (f32x16)(0.f);
      mfma_rows_x_frags<T, D>(sq, l32, hh, kf, s0, s1);
      mfma_rows_x_frags<T, D>(sdo, l32, hh, vf, d0, d1);

      // lane = key kkey; tile t register r = query qb0 + 32hh + 16t + r
      f32x16 pp0, pp1;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int qi = 32 * hh + 16 * t + r;
          const int q = qb0 + qi;
          const bool ok = kvalid && q < p.Sq && (!CAUSAL || kkey <= q);
          const float sx = t ? s1[r] : s0[r];
          const float dp = t ? d1[r] : d0[r];
          const float pv = ok ? exp2f(sx * p.scale_log2 - slse[qi]) : 0.f;
          const float ds = pv * (dp - sdl[qi]);
          if (t) { pp1[r] = pv; s1[r] = ds; } else { pp0[r] = pv; s0[r] = ds; }
        }
      Frag pfr[PF], dsf[PF];
      pack_frags<T>(pp0, pp1, pfr);
      pack_frags<T>(s0, s1, dsf);
      mfma_trn_x_frags<T, D>(sdot, l32, hh, pfr, dv);
      mfma_trn_x_frags<T, D>(sqt, l32, hh, dsf, dk);
    }
  }

  if (kkey < p.Sk) {
    store_acc_row<T, D>(static_cast<T*>(p.dk) + (koff + kkey) * D, dk, p.sm_scale, hh);
    store_acc_row<T, D>(static_cast<T*>(p.dv) + (koff + kkey) * D, dv, 1.f, hh);
  }
}

template <typename T, int D>
hipError_t delta_typed(const BwdParams& p, hipStream_t st) {
  constexpr int LPR = D / (16 / (int)sizeof(T));
  constexpr int RPB = 256 / LPR;
  const int64_t rows = (int64_t)p.B * p.Hq * p.Sq;
  hipLaunchKernelGGL((pf_attn_bwd_delta_kernel<T, D>), dim3((unsigned)((rows + RPB - 1) / RPB)), dim3(256),
                     0, st, p);
  return hipGetLastError();
}

template <typename T, int D>
hipError_t dq_typed(const BwdParams& p, bool causal, hipStream_t st) {
  const int n_qblk = (p.Sq + 127) / 128;
  const int n_work = p.B * p.Hq * n_qblk;
  if (causal)
    hipLaunchKernelGGL((pf_attn_bwd_dq_kernel<T, D, true>), dim3(n_work), dim3(256), 0, st, p, n_qblk, n_work);
  else
    hipLaunchKernelGGL((pf_attn_bwd_dq_kernel<T, D, false>), dim3(n_work), dim3(256), 0, st, p, n_qblk, n_work);
  return hipGetLastError();
}

template <typename T, int D>
hipError_t dkv_typed(const BwdParams& p, bool causal, hipStream_t st) {
  const int n_kblk = (p.Sk + 127) / 128;
  const int n_work = p.B * p.Hkv * n_kblk;
  if (causal)
    hipLaunchKernelGGL((pf_attn_bwd_dkv_kernel<T, D, true>), dim3(n_work), dim3(256), 0, st, p, n_kblk);
  else
    hipLaunchKernelGGL((pf_attn_bwd_dkv_kernel<T, D, false>), dim3(n_work), dim3(256), 0, st, p, n_kblk);
  return hipGetLastError();
}

#define PF_DISPATCH(FN, ...)                                                   \
  do {                                                                         \
    if (head_dim == 128) {                                                     \
      if (dtype == kF32) return FN<float, 128>(__VA_ARGS__);                   \
      if (dtype == kBF16) return FN<bf16_t, 128>(__VA_ARGS__);                 \
      if (dtype == kF16) return FN<f16_t, 128>(__VA_ARGS__);                   \
    } else if (head_dim == 64) {                                               \
      if (dtype == kF32) return FN<float, 64>(__VA_ARGS__);                    \
      if (dtype == kBF16) return FN<bf16_t, 64>(__VA_ARGS__);                  \
      if (dtype == kF16) return FN<f16_t, 64>(__VA_ARGS__);                    \
    }                                                                          \
    return hipErrorInvalidValue;                                               \
  } while (0)

}  // namespace

hipError_t launch_attn_bwd_delta(const BwdParams& p, int dtype, int head_dim, hipStream_t stream) {
  PF_DISPATCH(delta_typed, p, stream);
}

hipError_t launch_attn_bwd_dq(const BwdParams& p, int dtype, int head_dim, bool causal,
                              hipStream_t stream) {
  PF_DISPATCH(dq_typed, p, causal, stream);
}

hipError_t launch_attn_bwd_dkv(const BwdParams& p, int dtype, int head_dim, bool causal,
                               hipStream_t stream) {
  PF_DISPATCH(dkv_typed, p, causal, stream);
}

}  // namespace pf
