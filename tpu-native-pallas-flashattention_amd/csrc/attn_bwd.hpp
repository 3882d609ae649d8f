// Backward attention for gfx950: dQ kernel (which also computes delta),
// dK/dV kernel, and a standalone delta kernel for pf_attn_bwd_delta.
//
// Replaces `_flash_attention_bwd_call` (flash_attention.py:354-442):
//   delta_i = sum_d o_id * do_id            (XLA op, :363-365) -> in the dQ
//                                            kernel (or the delta kernel)
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
// Both kernels use the forward's pipeline: 64-row LDS tiles staged with
// bounds-checked buffer loads, double-buffered with one barrier per step, and
// every transposed operand read from the single natural copy with the
// transposing LDS load (pf_tiles.hpp).
//  dQ (workgroup = 128 query rows, 4 waves x 32 rows; loop over 64-key blocks;
//  it also computes delta for its rows and stores it for dK/dV):
//    S^T = K Q^T, dP^T = V dO^T  (K, V tiles; Q, dO in registers)
//    dS^T = P^T (dP^T - delta);  dQ^T += K^T dS^T  (K^T from the K tile)
//  dK/dV (workgroup = 128 keys, 4 waves x 32 keys; loop over the group's
//  heads x 64-row query blocks):
//    S = Q K^T, dP = dO V^T  (Q, dO tiles; K, V in registers)
//    dS = P (dP - delta);  dV^T += dO^T P,  dK^T += Q^T dS  (from the same tiles)
#pragma once

#include "pf_common.hpp"
#include "pf_kernels.hpp"
#include "pf_tiles.hpp"

#include <type_traits>

namespace pf {
namespace bwd {

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
__global__ __launch_bounds__(256, (kWgPerCu<T, D>))
void pf_attn_bwd_dq_kernel(BwdParams p, int n_qblk, int n_work) {
  using MF = Mfma32<T>;
  using Frag = typename MF::Frag;
  using G = Tile<T, D>;
  constexpr int BM = 128, BN = 64;
  constexpr int QF = (D / 2) / MF::kK;
  constexpr int NDT = D / 32;
  constexpr int PF = 32 / MF::kK;

  // two buffers x (K tile, V tile)
  __shared__ __attribute__((aligned(16))) char smem[4 * G::BYTES];

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, hh = lane >> 5, l32 = lane & 31;
  const int item = work_tail_item(p.tail, n_work, reinterpret_cast<int*>(smem));
  if (item < 0) return;
  const int w = xcd_remap(item, n_work, p.g);
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

  const int64_t qoff = (int64_t)(b * p.Hq + h) * p.Sq;
  const T* Qb = static_cast<const T*>(p.q) + qoff * D;
  const T* dOb = static_cast<const T*>(p.dout) + qoff * D;
  const T* Kb = static_cast<const T*>(p.k) + (int64_t)(b * p.Hkv + kvh) * p.Sk * D;
  const T* Vb = static_cast<const T*>(p.v) + (int64_t)(b * p.Hkv + kvh) * p.Sk * D;

  Frag qf[QF], dof[QF];
  load_row_frags<T, D>(Qb, qrow, qvalid, hh, qf);
  load_row_frags<T, D>(dOb, qrow, qvalid, hh, dof);
  const float lse2 = qvalid ? p.lse[qoff + qrow] * kLog2e : 0.f;
  // delta = sum_d f32(o) f32(do) of this row from the stored output
  // (flash_attention.py:363-365): each lane half sums its half of the row,
  // one exchange adds the two. Written for the dK/dV kernel, which runs
  // after this one.
  float dlt;
  {
    constexpr int EPC = 16 / (int)sizeof(T), FPC = frags_per_chunk<T>();
    const T* orow = static_cast<const T*>(p.o) + (qoff + (qvalid ? qrow : 0)) * D + hh * (D / 2);
    float part = 0.f;
#pragma unroll
    for (int c = 0; c < D / 2 / EPC; ++c) {
      float a[EPC], d[EPC];
      chunk_to_f32<T>(ldg16(orow + c * EPC), a);
      if constexpr (sizeof(T) == 4) {
#pragma unroll
        for (int f = 0; f < FPC; ++f) d[f] = dof[c * FPC + f];
      } else {
        chunk_to_f32<T>(__builtin_bit_cast(u32x4, dof[c]), d);
      }
#pragma unroll
      for (int e = 0; e < EPC; ++e) part += a[e] * d[e];
    }
    dlt = qvalid ? wave_xor32_sum(part) : 0.f;
    if (qvalid && hh == 0) p.delta[qoff + qrow] = dlt;
  }

  f32x16 acc[NDT];
#pragma unroll
  for (int i = 0; i < NDT; ++i) acc[i] = (f32x16)(0.f);

  const uint32_t kv_bytes = (uint32_t)p.kv_len * (uint32_t)G::RB;
  const i32x4 krs = make_desc(Kb, kv_bytes);
  const i32x4 vrs = make_desc(Vb, kv_bytes);
  TileDma<T, D> dma;
  dma.init(tid);
  TrAddr<T, D> kta;
  kta.init(lane);

  int kv_end = p.kv_len;
  if constexpr (CAUSAL) kv_end = min(kv_end, min(q0 + BM, p.Sq));
  const int nblk = (kv_end + BN - 1) / BN;

  if (nblk > 0) {
    dma.load(krs, 0, smem);
    dma.load(vrs, 0, smem + G::BYTES);
  }
  dma_wait();
  __syncthreads();

  // Key blocks in two straight-line loops: the leading run that needs no mask
  // for any wave of the workgroup (below the causal diagonal, inside kv_len,
  // all rows inside Sq), then the rest (diagonal, kv_len tail) with the mask.
  // Every wave runs every block: one whose keys are all masked for its rows
  // adds exact zeros (dS = 0).
  int n_plain = (q0 + BM > p.Sq) ? 0 : min(nblk, p.kv_len / BN);
  if constexpr (CAUSAL) n_plain = min(n_plain, q0 / BN);

  // Valid keys of this lane's query: key < klim (kv_len, and causal key <= q).
  const int klim = qvalid ? (CAUSAL ? min(p.kv_len, qrow + 1) : p.kv_len) : 0;
  auto block = [&](auto masked, int j) {
    const int kv0 = j * BN;
    // masked blocks: bit 16t + r says whether key kv0 + 32hh + 16t + r is valid
    uint32_t vmask = 0u;
    if constexpr (decltype(masked)::value) vmask = bit_range(0, klim - kv0 - 32 * hh);
    const char* sk = smem + (j & 1) * (2 * G::BYTES);
    const char* sv = sk + G::BYTES;
    if (j + 1 < nblk) {
      char* nk = smem + ((j + 1) & 1) * (2 * G::BYTES);
      dma.load(krs, kv0 + BN, nk);
      dma.load(vrs, kv0 + BN, nk + G::BYTES);
    }
    // keys kv0 + 32hh + 16t + r, query qrow.
    if constexpr (sizeof(T) == 2) {
      // One fenced sequence of four phases: S/dP half 0 (NS MFMAs) | S/dP
      // half 1 + P/dS VALU of half 0 | dQ half 0 (NQ MFMAs) + P/dS VALU of
      // half 1 | dQ half 1. LDS operands are read LEAD MFMAs ahead, across
      // the phase boundaries (global MFMA index g; phase starts 0, NS, 2NS,
      // 2NS + NQ).
      constexpr int NC = G::CPR / 2, NS = G::CPR, NQ = 2 * NDT, LEAD = 2, RING = 4;
      constexpr int NTOT = 2 * NS + 2 * NQ;
      typedef short v4i16 __attribute__((ext_vector_type(4)));
      const int rs0 = mfma_src_row(l32, 0), rs1 = mfma_src_row(l32, 1);
      const int sw0 = tile_swz<G::CPR>(rs0), sw1 = tile_swz<G::CPR>(rs1);
      f32x16 sx[2], dx[2];
      uint32_t dw[2][8];
      Frag opnd[RING];
      Frag dsf[2];
      // The dP chains start at -delta (this lane's query), so they end as
      // dP - delta and dS = P (dP - delta) needs no subtraction; the S chains
      // start from a literal zero (an inline constant of their first MFMA).
      dx[0] = dx[1] = (f32x16)(-dlt);
      // value r of half t: dS = P (dP - delta), pairs packed
      auto pds = [&](auto tc, int r) __attribute__((always_inline)) {
        constexpr int t = decltype(tc)::value;
        float pv = __builtin_amdgcn_exp2f(fmaf(sx[t][r], p.scale_log2, -lse2));
        if constexpr (decltype(masked)::value) pv = keep_if_bit(pv, vmask, 16 * t + r);
        sx[t][r] = pv * dx[t][r];
        if (r & 1) dw[t][r >> 1] = pack2<T>(sx[t][r - 1], sx[t][r]);
      };
      auto read = [&](int g) __attribute__((always_inline)) {
        if (g < 2 * NS) {
          // S/dP: k even = K chunk k/2 (S chain), k odd = V chunk k/2 (dP chain)
          const int t = g / NS, k = g % NS;
          const int r = t ? rs1 : rs0, sw = t ? sw1 : sw0;
          const char* tile = (k & 1) ? sv : sk;
          opnd[g % RING] = __builtin_bit_cast(Frag, lds16(tile + r * G::RB + 16 * ((hh * NC + (k >> 1)) ^ sw)));
        } else {
          // dQ: K^T step c = 2t + k / NDT, column block k % NDT
          const int t = (g - 2 * NS) / NQ, k = (g - 2 * NS) % NQ, c = 2 * t + k / NDT, dt = k % NDT;
          v4i16 part[2];
#pragma unroll
          for (int r = 0; r < 2; ++r)
            part[r] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) v4i16*)(sk + kta.off[dt][r] + (8 * c + 4 * r) * G::RB));
          opnd[g % RING] = __builtin_bit_cast(Frag, __builtin_shufflevector(part[0], part[1], 0, 1, 2, 3, 4, 5, 6, 7));
        }
      };
      // phase PH (compile-time): MFMAs g in [g0, g0 + n) with P/dS values
      // [v0, v0 + nv) of half vt (-1: none) spread over slots [SK, NS) of
      // the phase. dQ phases build each dS fragment right before its first
      // MFMA, so half 1's second fragment (values 8..15) can be computed
      // beside the first MFMAs of its own dQ phase.
      auto phase = [&](auto phc, auto vtc, auto v0c, auto nvc, auto skc, auto sec) __attribute__((always_inline)) {
        constexpr int ph = decltype(phc)::value, vt = decltype(vtc)::value;
        constexpr int v0 = decltype(v0c)::value, nv = decltype(nvc)::value;
        constexpr int SK = decltype(skc)::value, SE = decltype(sec)::value;
        constexpr int g0 = ph < 2 ? ph * NS : 2 * NS + (ph - 2) * NQ, n = ph < 2 ? NS : NQ;
#pragma unroll
        for (int k = 0; k < n; ++k) {
          const int g = g0 + k;
          if (g + LEAD < NTOT) read(g + LEAD);
          const Frag& a = opnd[g % RING];
          if constexpr (ph < 2) {
            if (k & 1) dx[ph] = MF::run(a, dof[k >> 1], dx[ph]);
            else sx[ph] = MF::run(a, qf[k >> 1], k == 0 ? (f32x16)(0.f) : sx[ph]);
          } else {
            constexpr int t = ph - 2;
            if (k % NDT == 0) {
              const int f = k / NDT;
              dsf[f] = __builtin_bit_cast(Frag, (u32x4){dw[t][4 * f], dw[t][4 * f + 1], dw[t][4 * f + 2], dw[t][4 * f + 3]});
            }
            acc[k % NDT] = MF::run(a, dsf[k / NDT], acc[k % NDT]);
          }
          if constexpr (vt >= 0) {
            if (k >= SK && k < SE) {
#pragma unroll
              for (int r = ((k - SK) * nv) / (SE - SK); r < ((k + 1 - SK) * nv) / (SE - SK); ++r)
                pds(std::integral_constant<int, vt>{}, v0 + r);
            }
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      };
#pragma unroll
      for (int g = 0; g < LEAD; ++g) read(g);
      __builtin_amdgcn_sched_barrier(0);
      using I = std::integral_constant<int, 0>;
      using IM = std::integral_constant<int, -1>;
      // half 1's S/dP chain ends just before phase 2: its P/dS starts two
      // slots in; values 8..15 must be done before slot NDT of phase 3
      phase(I{}, IM{}, I{}, I{}, I{}, I{});
      phase(std::integral_constant<int, 1>{}, I{}, I{}, std::integral_constant<int, 16>{}, I{},
            std::integral_constant<int, NS>{});
      phase(std::integral_constant<int, 2>{}, std::integral_constant<int, 1>{}, I{}, std::integral_constant<int, 8>{},
            std::integral_constant<int, 2>{}, std::integral_constant<int, NQ>{});
      phase(std::integral_constant<int, 3>{}, std::integral_constant<int, 1>{}, std::integral_constant<int, 8>{},
            std::integral_constant<int, 8>{}, I{}, std::integral_constant<int, NDT>{});
      dma_wait();
      __syncthreads();
      return;
    }
    // The two 32-key halves t are processed one after the other to keep
    // S^T/dP^T register use small.
    auto half = [&](auto tc) {
      constexpr int t = decltype(tc)::value;
      f32x16 sx = (f32x16)(0.f), dx = (f32x16)(0.f);
      mfma_nat_pair<T, D>(sk, qf, sv, dof, t, l32, hh, sx, dx);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float pv = __builtin_amdgcn_exp2f(fmaf(sx[r], p.scale_log2, -lse2));
        if constexpr (decltype(masked)::value) pv = keep_if_bit(pv, vmask, 16 * t + r);
        sx[r] = pv * (dx[r] - dlt);
      }
      // pack_frags(x, x) puts this half's fragments in both slot ranges;
      // steps [2t, 2t + 2) read the range of half t.
      Frag dsf[PF];
      pack_frags<T>(sx, sx, dsf);
      mfma_trn<T, D, 2 * t, 2 * t + 2>(sk, lane, kta, dsf, acc);
    };
    half(std::integral_constant<int, 0>{});
    half(std::integral_constant<int, 1>{});
    dma_wait();
    __syncthreads();
  };
  for (int j = 0; j < n_plain; ++j) block(std::false_type{}, j);
  for (int j = n_plain; j < nblk; ++j) block(std::true_type{}, j);

  if (qvalid) store_acc_row<T, D>(static_cast<T*>(p.dq) + (qoff + qrow) * D, acc, p.sm_scale, hh);
}

// ---------------------------------------------------------------------------
// dK / dV (group-summed)
// ---------------------------------------------------------------------------

// Order of the first S/dP phase of a dK/dV pass: position k of its 2n MFMAs
// runs S chunk op (op >= 0) or dP chunk -op - 1 (op < 0). The first dly + 1
// positions are S MFMAs, then the chains alternate, and whichever is left
// finishes the phase: the dP chain, which starts from -delta read from LDS at
// the top of the pass, then issues its first MFMA dly + 2 slots after that
// read instead of one. Each chain keeps its chunk order, so the sums are the
// same bit for bit.
__host__ __device__ constexpr int dkv_phase0_op(int k, int n, int dly) {
  int s = 0, d = 0;
  for (int pos = 0; pos <= k; ++pos) {
    bool take_s;
    if (s == n) take_s = false;
    else if (d == n) take_s = true;
    else if (s <= dly) take_s = true;
    else take_s = (pos - (dly + 1)) % 2 == 1;
    if (pos == k) return take_s ? s : -(d + 1);
    if (take_s) ++s;
    else ++d;
  }
  return 0;
}
template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void pf_attn_bwd_dkv_kernel(BwdParams p, int n_kblk) {
  using MF = Mfma32<T>;
  using Frag = typename MF::Frag;
  using G = Tile<T, D>;
  // A step covers BMQ query rows of one head as NSUB sub-steps of 64 rows;
  // 16-bit up to head_dim 128: 128 rows, so the per-step work (tile DMA
  // issue, lse/delta staging, DMA wait, barrier) is shared by two sub-steps,
  // and the step runs as one fenced MFMA sequence with the dK/dV
  // accumulators in AGPRs (kAcc). float32, and 16-bit at head_dim 256
  // (whose 128-row double buffer would exceed the LDS and whose dK/dV
  // accumulators alone fill the AGPRs): 64 rows with the plain step body.
  constexpr bool kAcc = sizeof(T) == 2 && D <= 128;
  constexpr int BNK = 128, BMQ = kAcc ? 128 : 64, NSUB = BMQ / 64;
  constexpr int KF = (D / 2) / MF::kK;
  constexpr int NDT = D / 32;
  constexpr int PF = 32 / MF::kK;
  // dK/dV columns one workgroup accumulates: all D, or at head_dim 256 the
  // 128-column half blockIdx.y selects (S and dP still contract over all D,
  // so the two workgroups of a key block both compute them). The half's
  // transposed reads are those of the first half 256 bytes further on: the
  // tile swizzle permutes only the low 16 chunks (256 bytes) of a row.
  constexpr int DA = D > 128 ? 128 : D, NDA = DA / 32;
  static_assert(!kAcc || DA == D, "the fenced sequence accumulates every column");
  static_assert(DA == D || (DA * (int)sizeof(T)) % 256 == 0, "column halves above the swizzled chunks");
  const int dcol = DA == D ? 0 : (int)blockIdx.y * DA;

  // two buffers x (Q sub-tiles [NSUB], dO sub-tiles [NSUB], lse[BMQ], delta[BMQ])
  constexpr int BUF = 2 * NSUB * G::BYTES + 2 * BMQ * 4;
  __shared__ __attribute__((aligned(16))) char smem[2 * BUF];

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

  f32x16 dk[NDA], dv[NDA];
#pragma unroll
  for (int i = 0; i < NDA; ++i) {
    dk[i] = (f32x16)(0.f);
    dv[i] = (f32x16)(0.f);
  }

  const int q_begin = CAUSAL ? (k0 / BMQ) * BMQ : 0;
  const int nqb = (k0 < p.kv_len && q_begin < p.Sq) ? (p.Sq - q_begin + BMQ - 1) / BMQ : 0;
  const int nsteps = nqb * p.g;  // (group member, q block) pairs

  // Step order: every step that needs a mask for some wave of the workgroup
  // first, then the rest (order below), so each of the two loops has one straight-
  // line body (a branch between masked and unmasked bodies would merge the
  // dK/dV accumulators across blocks and cost register-file copies).
  // Masked: the causal diagonal blocks (query block start < k0 + BNK - 1),
  // the last query block when Sq is ragged, or every block when the
  // workgroup's keys cross kv_len.
  const bool all_masked = k0 + BNK > p.kv_len;
  const int nd = CAUSAL ? min(nqb, (k0 + BNK - 1 - q_begin + BMQ - 1) / BMQ) : 0;
  const int tail = ((p.Sq - q_begin) % BMQ != 0 && nqb > nd) ? 1 : 0;
  const int m_pm = all_masked ? nqb : nd + tail;  // masked blocks per member
  const int u_pm = nqb - m_pm;                     // unmasked blocks per member
  const int n_masked = m_pm * p.g;

  float lreg = 0.f;  // threads 0..63 stage lse, 64..127 stage delta
  TrAddr<T, D> ta;
  ta.init(lane);

  // Step st -> (query head h, query block start qb0), tracked incrementally
  // (no integer division in the loop): position (a, c) is (member, masked
  // block index k) while st < n_masked, then (member, descending block index).
  struct Pos {
    int a, c;
  };
  auto coords = [&](int st, Pos ps, int& h, int& qb0) {
    int blk;
    if (st < n_masked) {
      blk = (all_masked || ps.c < nd) ? ps.c : nqb - 1;
    } else {
      // Unmasked steps: query blocks from the last one down (outer), group
      // members inner. Workgroups of one (b, kv head) share an XCD and all
      // start at the top block, so at any time they stream the same Q/dO
      // tiles and read them mostly from that XCD's L2.
      blk = nd + (u_pm - 1 - ps.c);
    }
    h = kvh * p.g + ps.a;
    qb0 = q_begin + blk * BMQ;
  };
  // position of step st + 1 from that of step st
  auto advance = [&](int st, Pos ps) -> Pos {
    if (st + 1 < n_masked) {
      if (++ps.c == m_pm) {
        ps.c = 0;
        ++ps.a;
      }
      return ps;
    }
    if (st + 1 == n_masked) return Pos{0, 0};
    if (++ps.a == p.g) {
      ps.a = 0;
      ++ps.c;
    }
    return ps;
  };
  TileDma<T, D> dma;
  dma.init(tid);
  const int wv_u = __builtin_amdgcn_readfirstlane(wv);  // wave index, known uniform
  auto load_step = [&](int h, int qb0, char* buf) {
    const int64_t qoff = (int64_t)(b * p.Hq + h) * p.Sq;
    const uint32_t qbytes = (uint32_t)p.Sq * (uint32_t)G::RB;
    const i32x4 qd = make_desc(static_cast<const T*>(p.q) + qoff * D, qbytes);
    const i32x4 dd = make_desc(static_cast<const T*>(p.dout) + qoff * D, qbytes);
#pragma unroll
    for (int u = 0; u < NSUB; ++u) {
      dma.load(qd, qb0 + 64 * u, buf + u * G::BYTES);
      dma.load(dd, qb0 + 64 * u, buf + (NSUB + u) * G::BYTES);
    }
    // Raw load only: a use here would make the wave wait (vmcnt(0)) for the
    // tile DMA just issued as well; the log2 scaling happens at the store.
    // The first BMQ/64 waves stage lse, the next BMQ/64 delta (a wave-uniform
    // choice: the pointer stays in scalar registers).
    const int q = min(qb0 + (tid & (BMQ - 1)), p.Sq - 1);
    if (wv_u < 2 * NSUB) lreg = (wv_u < NSUB ? p.lse : p.delta)[qoff + q];
  };
  // LDS holds lse in log2 units and -delta (the dP chains start from it).
  auto store_step = [&](char* buf, int qb0) {
    if (tid < 2 * BMQ) {
      const bool valid = qb0 + (tid & (BMQ - 1)) < p.Sq;
      reinterpret_cast<float*>(buf + 2 * NSUB * G::BYTES)[tid] = valid ? (tid < BMQ ? lreg * kLog2e : -lreg) : 0.f;
    }
  };

  Pos pos{0, 0};  // of step 0 (a masked or an unmasked step alike)
  if (nsteps > 0) {
    int h0, qb00;
    coords(0, pos, h0, qb00);
    load_step(h0, qb00, smem);
    store_step(smem, qb00);
  }
  dma_wait();
  __syncthreads();

  // One step: lane = key kkey; half t register r = query qb0 + 32hh + 16t + r.
  // P = exp2(S c - lse) (masked to 0), dS = P (dP - delta); then
  // dV^T += dO^T P and dK^T += Q^T dS. Every wave runs every step: one whose
  // keys are all masked for it (past kv_len, causal rows all above its keys)
  // adds exact zeros (P = dS = 0).
  // 16-bit: at one wave per SIMD nothing else hides a stall, so the step is
  // one fenced MFMA sequence with LDS operands read two MFMAs ahead, in four
  // phases: S/dP half 0 | S/dP half 1 + P/dS VALU of half 0 |
  //   dV/dK of half 0 + P/dS VALU of half 1 | dV/dK of half 1.
  // 16-bit: operand ring of the fenced sequence, shared by the NSUB passes
  // of a step so that the last slots of one pass can read the first operands
  // of the next (its Q/dO sub-tiles are already resident).
  typename MF::Frag opnd[3];
  auto step_body = [&](auto masked, auto uc, const char* sq, const char* sdo, const float* slse, const float* sdl,
                       int qb0) {
    constexpr int U = decltype(uc)::value;  // pass within the step
    // Masked steps: value (half t, register r) of this lane is query
    // qb0 + 32hh + 16t + r against key kkey; bit 16t + r of vmask says whether
    // it is valid (key < kv_len, query < Sq, causal key <= query).
    uint32_t vmask = 0u;
    if constexpr (decltype(masked)::value) {
      const int base = qb0 + 32 * hh;
      vmask = kvalid ? bit_range(CAUSAL ? kkey - base : 0, p.Sq - base) : 0u;
    }
    f32x16 sx[2], dx[2];
    if constexpr (kAcc) {
      f32x4 lv[2][4], dl[2][4];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          lv[t][r4] = reinterpret_cast<const f32x4*>(slse + 32 * hh + 16 * t)[r4];
          dl[t][r4] = reinterpret_cast<const f32x4*>(sdl + 32 * hh + 16 * t)[r4];
        }
      uint32_t pw[2][8], dw[2][8];
      Frag pf[2][2], df[2][2];
      using H0 = std::integral_constant<int, 0>;
      using H1 = std::integral_constant<int, 1>;
      constexpr int NP = G::CPR;
      // value r of half t: P overwrites S and dS overwrites dP; pairs packed.
      auto pds = [&](auto tc, int r) {
        constexpr int t = decltype(tc)::value;
        float pv = __builtin_amdgcn_exp2f(fmaf(sx[t][r], p.scale_log2, -lv[t][r >> 2][r & 3]));
        if constexpr (decltype(masked)::value) pv = keep_if_bit(pv, vmask, 16 * t + r);
        const float ds = pv * dx[t][r];
        sx[t][r] = pv;
        dx[t][r] = ds;
        if (r & 1) {
          pw[t][r >> 1] = pack2<T>(sx[t][r - 1], pv);
          dw[t][r >> 1] = pack2<T>(dx[t][r - 1], ds);
        }
      };
      auto frags = [&](const uint32_t* w, Frag* f) {
        f[0] = __builtin_bit_cast(Frag, (u32x4){w[0], w[1], w[2], w[3]});
        f[1] = __builtin_bit_cast(Frag, (u32x4){w[4], w[5], w[6], w[7]});
      };
      // D = 128 (one value per MFMA slot): the P/dS work of each value is
      // software-pipelined over three slots -- FMA in slot NP (1 + t) + r,
      // exp2 (and mask) one slot later, dS, the stores and the packing two
      // slots later -- so no VALU op waits on a result of its own slot (at
      // one wave per SIMD nothing else would fill that wait). The last values
      // of a half finish in the first two slots of the next phase; their
      // fragment (values 8..15) is first read 2 NDT slots into that phase.
      constexpr bool kPipe = (G::CPR == 16);
      float ya[2][16], pe[2][16];
      auto stage = [&](auto tc, auto stc, int r) __attribute__((always_inline)) {
        constexpr int t = decltype(tc)::value, st = decltype(stc)::value;
        if constexpr (st == 0) {
          ya[t][r] = fmaf(sx[t][r], p.scale_log2, -lv[t][r >> 2][r & 3]);
          asm volatile("" : "+v"(ya[t][r]));
        } else if constexpr (st == 1) {
          float pv = __builtin_amdgcn_exp2f(ya[t][r]);
          if constexpr (decltype(masked)::value) pv = keep_if_bit(pv, vmask, 16 * t + r);
          pe[t][r] = pv;
          asm volatile("" : "+v"(pe[t][r]));
        } else {
          const float pv = pe[t][r];
          const float ds = pv * dx[t][r];
          sx[t][r] = pv;
          dx[t][r] = ds;
          if (r & 1) {
            pw[t][r >> 1] = pack2<T>(sx[t][r - 1], pv);
            dw[t][r >> 1] = pack2<T>(dx[t][r - 1], ds);
            asm volatile("" : "+v"(pw[t][r >> 1]), "+v"(dw[t][r >> 1]));
          }
          if (r == 7) {
            pf[t][0] = __builtin_bit_cast(Frag, (u32x4){pw[t][0], pw[t][1], pw[t][2], pw[t][3]});
            df[t][0] = __builtin_bit_cast(Frag, (u32x4){dw[t][0], dw[t][1], dw[t][2], dw[t][3]});
          } else if (r == 15) {
            pf[t][1] = __builtin_bit_cast(Frag, (u32x4){pw[t][4], pw[t][5], pw[t][6], pw[t][7]});
            df[t][1] = __builtin_bit_cast(Frag, (u32x4){dw[t][4], dw[t][5], dw[t][6], dw[t][7]});
          }
        }
      };
      // the pipelined stages of global slot j
      auto pipe = [&](int j) __attribute__((always_inline)) {
        using S0 = std::integral_constant<int, 0>;
        using S1 = std::integral_constant<int, 1>;
        using S2 = std::integral_constant<int, 2>;
        const int r0 = j - NP, r1 = j - 2 * NP;  // value index of stage 0 per half
        if (r0 >= 0 && r0 < 16) stage(H0{}, S0{}, r0);
        if (r0 - 1 >= 0 && r0 - 1 < 16) stage(H0{}, S1{}, r0 - 1);
        if (r0 - 2 >= 0 && r0 - 2 < 16) stage(H0{}, S2{}, r0 - 2);
        if (r1 >= 0 && r1 < 16) stage(H1{}, S0{}, r1);
        if (r1 - 1 >= 0 && r1 - 1 < 16) stage(H1{}, S1{}, r1 - 1);
        if (r1 - 2 >= 0 && r1 - 2 < 16) stage(H1{}, S2{}, r1 - 2);
      };
      // One fenced sequence of 4 phases x NP MFMAs (NP = CPR): S/dP half 0,
      // S/dP half 1, dV/dK half 0, dV/dK half 1. Operands are read LEAD MFMAs
      // ahead, across phase boundaries too.
      constexpr int NC = G::CPR / 2, LEAD = 2;
      // delay of the half-0 dP chain in phase 0 (dkv_phase0_op)
      constexpr int kDpDelay = 3;
      // (is dP, chunk) of MFMA k of S/dP phase ph
      auto sdp_op = [&](int ph, int k, bool& dp, int& ch) __attribute__((always_inline)) {
        if (ph == 0) {
          const int op = dkv_phase0_op(k, NC, kDpDelay);
          dp = op < 0;
          ch = dp ? -op - 1 : op;
        } else {
          dp = (k & 1) != 0;
          ch = k >> 1;
        }
      };
      constexpr int VPS = 16 / NP;  // P/dS values per MFMA slot
      typedef short v4i16 __attribute__((ext_vector_type(4)));
      const int rs0 = mfma_src_row(l32, 0), rs1 = mfma_src_row(l32, 1);
      const int sw0 = tile_swz<G::CPR>(rs0), sw1 = tile_swz<G::CPR>(rs1);
      static_assert(LEAD + 1 == 3, "ring size");
      // MFMA i of pass U uses ring slot (ROFF + i) % 3: the index runs on
      // across the passes of a step
      constexpr int NT = 4 * NP, ROFF = (U * NT) % (LEAD + 1);
      // The dP chains start at -delta (per query = per register; staged
      // negated), so they end as dP - delta and dS = P (dP - delta) needs no
      // subtraction.
      sx[0] = sx[1] = (f32x16)(0.f);
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) dx[t][r] = dl[t][r >> 2][r & 3];
      // operand of MFMA i (i >= NT: MFMA i - NT of the next pass)
      auto read = [&](int i) __attribute__((always_inline)) {
        const int slot = (ROFF + i) % (LEAD + 1);
        const bool nx = i >= NT;
        const int ii = nx ? i - NT : i;
        const int ph = ii / NP, k = ii % NP;
        if (ph < 2) {
          // S/dP: Q chunk ch (S chain) or dO chunk ch (dP chain), in the
          // phase's order (sdp_op)
          bool dp;
          int ch;
          sdp_op(ph, k, dp, ch);
          const int r = ph ? rs1 : rs0, sw = ph ? sw1 : sw0;
          const char* tile = (dp ? sdo : sq) + (nx ? G::BYTES : 0);
          opnd[slot] = __builtin_bit_cast(Frag, lds16(tile + r * G::RB + 16 * ((hh * NC + ch) ^ sw)));
        } else {
          // dV/dK: k even = dO^T (dV), k odd = Q^T (dK); m = k/2: step 2t + m/NDT, block m%NDT
          const int t = ph - 2, m = k >> 1, c = 2 * t + m / NDT, dt = m % NDT;
          const char* tile = (k & 1) ? sq : sdo;
          v4i16 part[2];
#pragma unroll
          for (int r = 0; r < 2; ++r)
            part[r] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) v4i16*)(tile + ta.off[dt][r] + (8 * c + 4 * r) * G::RB));
          opnd[slot] =
              __builtin_bit_cast(Frag, __builtin_shufflevector(part[0], part[1], 0, 1, 2, 3, 4, 5, 6, 7));
        }
      };
      // Phase PH as its own unrolled loop (compile-time phase: every index
      // below is a constant); MFMA j's operand was read LEAD MFMAs earlier,
      // possibly in the previous phase.
      auto phase = [&](auto phc) __attribute__((always_inline)) {
        constexpr int ph = decltype(phc)::value;
#pragma unroll
        for (int k = 0; k < NP; ++k) {
          const int j = ph * NP + k;
          if (j + LEAD < NT || U + 1 < NSUB) read(j + LEAD);
          const Frag& a = opnd[(ROFF + j) % (LEAD + 1)];
          if constexpr (ph < 2) {
            bool dp;
            int ch;
            sdp_op(ph, k, dp, ch);
            if (dp) dx[ph] = MF::run(a, vf[ch], dx[ph]);
            else sx[ph] = MF::run(a, kf[ch], sx[ph]);
            if constexpr (ph == 1 && !kPipe) {
#pragma unroll
              for (int e = 0; e < VPS; ++e) pds(H0{}, k * VPS + e);
            }
          } else {
            constexpr int t = ph - 2;
            const int m = k >> 1, cc = m / NDT, dt = m % NDT;
            f32x16& acc = (k & 1) ? dk[dt] : dv[dt];
            const Frag& bf = (k & 1) ? df[t][cc] : pf[t][cc];
            if constexpr (kAcc) MfmaAgpr<T>::run(acc, a, bf);
            else acc = MF::run(a, bf, acc);
            if constexpr (ph == 2 && !kPipe) {
#pragma unroll
              for (int e = 0; e < VPS; ++e) pds(H1{}, k * VPS + e);
            }
          }
          if constexpr (kPipe) pipe(j);
          __builtin_amdgcn_sched_barrier(0);
        }
      };
      if constexpr (U == 0) {  // later passes had theirs read by the previous one
#pragma unroll
        for (int i = 0; i < LEAD; ++i) read(i);
      }
      __builtin_amdgcn_sched_barrier(0);
      phase(std::integral_constant<int, 0>{});
      phase(std::integral_constant<int, 1>{});
      if constexpr (!kPipe) {
        frags(pw[0], pf[0]);
        frags(dw[0], df[0]);
      }
      phase(std::integral_constant<int, 2>{});
      if constexpr (!kPipe) {
        frags(pw[1], pf[1]);
        frags(dw[1], df[1]);
      }
      phase(std::integral_constant<int, 3>{});
    } else {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        sx[t] = (f32x16)(0.f);
        dx[t] = (f32x16)(0.f);
        mfma_nat_pair<T, D>(sq, kf, sdo, vf, t, l32, hh, sx[t], dx[t]);
      }
      auto half = [&](auto tc) {
        constexpr int t = decltype(tc)::value;
        const f32x4* l4 = reinterpret_cast<const f32x4*>(slse + 32 * hh + 16 * t);
        const f32x4* d4 = reinterpret_cast<const f32x4*>(sdl + 32 * hh + 16 * t);
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const f32x4 lv = l4[r4], dl = d4[r4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = 4 * r4 + e;
            float pv = __builtin_amdgcn_exp2f(fmaf(sx[t][r], p.scale_log2, -lv[e]));
            if constexpr (decltype(masked)::value) pv = keep_if_bit(pv, vmask, 16 * t + r);
            dx[t][r] = pv * (dx[t][r] + dl[e]);  // dl = -delta
            sx[t][r] = pv;
          }
        }
        // pack_frags(x, x) puts this half's fragments in both slot ranges;
        // steps [2t, 2t + 2) read the range of half t.
        Frag pfr[PF], dsf[PF];
        pack_frags<T>(sx[t], sx[t], pfr);
        pack_frags<T>(dx[t], dx[t], dsf);
        const int cb = dcol * (int)sizeof(T);  // byte offset of the column half
        mfma_trn<T, D, 2 * t, 2 * t + 2, false, NDA>(sdo + cb, lane, ta, pfr, dv);
        mfma_trn<T, D, 2 * t, 2 * t + 2, false, NDA>(sq + cb, lane, ta, dsf, dk);
      };
      half(std::integral_constant<int, 0>{});
      half(std::integral_constant<int, 1>{});
    }
  };

  int st = 0;
  auto run = [&](auto masked, int st_end) {
    for (; st < st_end; ++st) {
      const char* buf = smem + (st & 1) * BUF;
      const float* slse = reinterpret_cast<const float*>(buf + 2 * NSUB * G::BYTES);
      int h_unused, qb0;
      coords(st, pos, h_unused, qb0);
      const Pos npos = advance(st, pos);
      int nh = 0, nqb0 = 0;
      const bool has_next = st + 1 < nsteps;
      if (has_next) coords(st + 1, npos, nh, nqb0);
      char* const nbuf = smem + ((st + 1) & 1) * BUF;
      if (has_next) load_step(nh, nqb0, nbuf);
      // one copy of the sequence per 64-row pass
      static_for<NSUB>([&](auto uc) __attribute__((always_inline)) {
        constexpr int u = decltype(uc)::value;
        step_body(masked, uc, buf + u * G::BYTES, buf + (NSUB + u) * G::BYTES, slse + 64 * u, slse + BMQ + 64 * u,
                  qb0 + 64 * u);
      });
      if (has_next) store_step(nbuf, nqb0);
      pos = npos;
      dma_wait();
      __syncthreads();
    }
  };
  run(std::true_type{}, n_masked);
  run(std::false_type{}, nsteps);

  if constexpr (kAcc) {
#pragma unroll
    for (int i = 0; i < NDA; ++i) {
      agpr_fence(dk[i]);
      agpr_fence(dv[i]);
    }
  }
  if (kkey < p.Sk) {
    store_acc_row<T, DA>(static_cast<T*>(p.dk) + (koff + kkey) * D + dcol, dk, p.sm_scale, hh);
    store_acc_row<T, DA>(static_cast<T*>(p.dv) + (koff + kkey) * D + dcol, dv, 1.f, hh);
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
  const int n_work = bwd_dq_items(p);
  const dim3 grid(work_tail_grid(p.tail, n_work));
  if (causal)
    hipLaunchKernelGGL((pf_attn_bwd_dq_kernel<T, D, true>), grid, dim3(256), 0, st, p, n_qblk, n_work);
  else
    hipLaunchKernelGGL((pf_attn_bwd_dq_kernel<T, D, false>), grid, dim3(256), 0, st, p, n_qblk, n_work);
  return hipGetLastError();
}

template <typename T, int D>
hipError_t dkv_typed(const BwdParams& p, bool causal, hipStream_t st) {
  const int n_kblk = (p.Sk + 127) / 128;
  // head_dim 256: two workgroups per key block, one per 128-column half of dK/dV
  const dim3 grid(bwd_dkv_items(p), D > 128 ? 2 : 1);
  if (causal)
    hipLaunchKernelGGL((pf_attn_bwd_dkv_kernel<T, D, true>), grid, dim3(256), 0, st, p, n_kblk);
  else
    hipLaunchKernelGGL((pf_attn_bwd_dkv_kernel<T, D, false>), grid, dim3(256), 0, st, p, n_kblk);
  return hipGetLastError();
}

}  // namespace bwd
}  // namespace pf
