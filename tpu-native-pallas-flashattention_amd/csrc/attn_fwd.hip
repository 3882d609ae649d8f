// Forward prefill attention for gfx950 (CDNA4), with optional fused RoPE
// (Q rotated in registers here; K rotated once by pf_rope_rotate_k_kernel).
//
// Replaces the reference's `flash_attention_fwd` pallas_call
// (flash_attention.py:162-227, kernel :61-159) and `flash_attention_rope_fwd`
// (fused_rope.py:183-213, kernel :53-113).
//
// Work decomposition: one workgroup of 4 waves per (batch, GQA head group,
// query block); each wave owns 32 query rows of one head. A workgroup packs
// hpw query heads of one GQA group (4 when the group size allows) x 128/hpw
// rows, so the K/V tiles it stages serve all those heads. The grid is 1-D: heavy (late) query
// blocks first for causal load balance, and the workgroups sharing a KV head
// on one XCD so they share K/V in that XCD's L2 (fwd_work_item).
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
// values V[k0 + t][d0 + i]). For float32 each lane reads its single V^T
// element of an MFMA step straight from the row-major tile.
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

#include <type_traits>

namespace pf {

namespace {

constexpr int kFwdBN = 64;   // keys per block


template <typename T, int D, bool CAUSAL, bool ROPE>
__global__ __launch_bounds__(256, (kWgPerCu<T, D>)) void pf_attn_fwd_kernel(FwdParams p) {
  using MF = Mfma32<T>;
  using Frag = typename MF::Frag;
  using G = Tile<T, D>;
  constexpr int BN = kFwdBN;
  constexpr int HALF = D / 2;
  constexpr int ES = G::ES, EPC = G::EPC;
  constexpr int FPC = frags_per_chunk<T>();
  constexpr int QF = HALF / MF::kK;  // Q fragments per lane
  constexpr int NDT = D / 32;        // 32-row tiles of O^T
  constexpr int PF = 32 / MF::kK;    // P fragments per lane per block
  static_assert(BN == 64, "one K/V block is one 64-row tile");

  // Fused RoPE, 16-bit, all four waves on the same 32 query rows (hpw = 4):
  // the workgroup's slice of the cos/sin tables (32 rows each, float32) is
  // staged in LDS by one coalesced DMA and each lane reads its row from
  // there. Loaded straight from global memory instead, every lane reads 512
  // contiguous bytes of its own row, so each load instruction touches 64
  // rows; those scattered loads, repeated by all four waves, were most of
  // the fused forward's extra time. The slice occupies V buffer 1 (not
  // loaded before the first block's barrier) and one more tile.
  constexpr bool kStageTab = ROPE && ES == 2;
  constexpr int kTabRows = 32;
  constexpr int kTabBytes = kTabRows * D * 4;  // one table's slice
  static_assert(!kStageTab || 2 * kTabBytes == 2 * G::BYTES, "table slices fill V buffer 1 + one tile");
  // two buffers x (K tile, V tile) [+ the table tile]
  __shared__ __attribute__((aligned(16))) char smem[(kStageTab ? 5 : 4) * G::BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int hh = lane >> 5;
  const int l32 = lane & 31;

  // work item = (batch, kv head, head group, query block); the workgroup's
  // waves split into hpw heads x (4 / hpw) 32-row slices.
  int b, kvh, hg, qblk;
  const int item = work_tail_item(p.tail, p.n_work, reinterpret_cast<int*>(smem));
  if (item < 0) return;
  fwd_work_item(item, p, b, kvh, hg, qblk);
  const int wph = 4 / p.hpw;  // waves per head
  const int h = kvh * p.g + hg * p.hpw + wv / wph;

  const int q0 = qblk * p.rpw;
  const int wq0 = q0 + 32 * (wv % wph);
  const int qrow = wq0 + l32;

  const T* Qb = static_cast<const T*>(p.q) + (int64_t)(b * p.Hq + h) * p.Sq * D;
  const T* Kb = static_cast<const T*>(p.k) + (int64_t)(b * p.Hkv + kvh) * p.Sk * D;
  const T* Vb = static_cast<const T*>(p.v) + (int64_t)(b * p.Hkv + kvh) * p.Sk * D;

  // ---- staging: K/V rows at or past kv_len lie outside the buffer resources
  // and load as zeros (never read from memory). K and V go global -> LDS by
  // DMA (with fused RoPE, p.k is the K rotated once by pf_rope_rotate_k_kernel).
  const uint32_t kv_bytes = (uint32_t)p.kv_len * (uint32_t)(D * ES);
  const i32x4 krs = make_desc(Kb, kv_bytes);
  const i32x4 vrs = make_desc(Vb, kv_bytes);
  TileDma<T, D> dma;
  dma.init(tid);
  int kv_end = p.kv_len;
  if constexpr (CAUSAL) kv_end = min(kv_end, min(q0 + p.rpw, p.Sq));
  const int nblk = (kv_end + BN - 1) / BN;
  // LDS: K tiles at [0, 2 BYTES) (block j in j & 1), V tiles after them.
  auto first_tiles = [&]() {
    if (nblk > 0) {
      dma.load(krs, 0, smem);
      dma.load(vrs, 0, smem + 2 * G::BYTES);
      if (nblk > 1) dma.load(krs, BN, smem + G::BYTES);
    }
  };
  // Without RoPE the first tiles are requested before Q, which only the
  // first block's MFMAs (after those tiles) need. With RoPE, Q and its table
  // rows go first: vmcnt counts loads in issue order, so the rotation would
  // otherwise wait for the tiles too.
  if constexpr (!ROPE) first_tiles();

  // ---- Q fragment (B operand of S^T): lane holds Q[qrow][hh*HALF, +HALF).
  // Rows past Sq load row 0 (in bounds; no branch around the loads) and are
  // zeroed after the wait.
  const bool qvalid = qrow < p.Sq;
  const bool stage_tab = kStageTab && p.hpw == 4;  // workgroup-uniform
  char* const tab = smem + 3 * G::BYTES;            // cos slice, then sin slice
  u32x4 qc[HALF / EPC];
  [[maybe_unused]] f32x4 ct[ROPE ? HALF / 4 : 1], st[ROPE ? HALF / 4 : 1];
  {
    const T* qr = Qb + (int64_t)(qvalid ? qrow : 0) * D + hh * HALF;
#pragma unroll
    for (int c = 0; c < HALF / EPC; ++c) qc[c] = ldg16(qr + c * EPC);
    if constexpr (ROPE) {
      if (stage_tab) {
        // Table row q0 + r lands at tab + r * 4D with its 16-byte chunk ch at
        // position ch ^ (r & 15): the 16 lanes of an LDS read (16 rows, one
        // chunk index) then hit 16 different bank groups. Rows past Sq lie
        // outside the descriptors and arrive as zeros.
        constexpr int CPRT = D / 4;  // 16-byte chunks per table row
        constexpr int PER = kTabRows * CPRT / 256;
        const uint32_t nb = (uint32_t)max(0, min(kTabRows, p.Sq - q0)) * (uint32_t)(D * 4);
        const i32x4 cd = make_desc(p.q_cos + (int64_t)q0 * D, nb);
        const i32x4 sd = make_desc(p.q_sin + (int64_t)q0 * D, nb);
        const int w = __builtin_amdgcn_readfirstlane(wv);
#pragma unroll
        for (int u = 0; u < PER; ++u) {
          const int slot = 64 * (4 * u + w) + lane;  // 16-byte slot within a slice
          const int r = slot / CPRT, pos = slot % CPRT;
          const uint32_t voff = (uint32_t)(r * D * 4 + 16 * (pos ^ (r & 15)));
          const uint32_t la = __builtin_amdgcn_readfirstlane(lds_u32(tab) + 16 * 64 * (4 * u + w));
          dma16(cd, voff, la);
          dma16(sd, voff, la + kTabBytes);
        }
      } else {
        const float* cr = p.q_cos + (int64_t)(qvalid ? qrow : 0) * D + hh * HALF;
        const float* sr = p.q_sin + (int64_t)(qvalid ? qrow : 0) * D + hh * HALF;
#pragma unroll
        for (int c = 0; c < HALF / 4; ++c) {
          ct[c] = *reinterpret_cast<const f32x4*>(cr + 4 * c);
          st[c] = *reinterpret_cast<const f32x4*>(sr + 4 * c);
        }
      }
    }
  }

  if constexpr (ROPE) first_tiles();

  Frag qf[QF];
  {
    if (!qvalid) {
#pragma unroll
      for (int c = 0; c < HALF / EPC; ++c) qc[c] = (u32x4){0u, 0u, 0u, 0u};
    }
    if constexpr (ROPE) {
      if (stage_tab) {
        // The table DMA went out before the K/V tiles' (3 tiles of
        // TileDma::PER_T loads per lane at most): wait for it alone, then for
        // every wave's part of it.
        constexpr int KV_LOADS = TileDma<T, D>::PER_T;
        if (nblk > 1) wait_vm<3 * KV_LOADS>();
        else wait_vm<2 * KV_LOADS>();
        __syncthreads();
        const int r = l32;  // the lane's row within the slice (wq0 == q0 here)
#pragma unroll
        for (int c = 0; c < HALF / 4; ++c) {
          const int ch = hh * (HALF / 4) + c;
          const char* a = tab + r * D * 4 + 16 * (ch ^ (r & 15));
          ct[c] = __builtin_bit_cast(f32x4, lds16(a));
          st[c] = __builtin_bit_cast(f32x4, lds16(a + kTabBytes));
        }
      }
      // x*cos + rotate_half(x)*sin in float32 (fused_rope.py:43-50, :75-78):
      // element d of half hh is x[d] cos[d] - x[d + HALF] sin[d] (hh = 0) or
      // x[d] cos[d] + x[d - HALF] sin[d] (hh = 1); the partner half lives in
      // lane l ^ 32 and is exchanged with v_permlane32_swap (which returns
      // the pair's two values; partner = both ^ own, whatever their order).
      const float sgn = hh ? 1.f : -1.f;
#pragma unroll
      for (int c = 0; c < HALF / EPC; ++c) {
        u32x4 pc;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const auto r = __builtin_amdgcn_permlane32_swap(qc[c][w], qc[c][w], false, false);
          pc[w] = r[0] ^ r[1] ^ qc[c][w];
        }
        float x[EPC], xp[EPC], y[EPC];
        chunk_to_f32<T>(qc[c], x);
        chunk_to_f32<T>(pc, xp);
#pragma unroll
        for (int e = 0; e < EPC; ++e) {
          const int i = c * EPC + e;  // element within the half
          y[e] = x[e] * ct[i / 4][i % 4] + sgn * xp[e] * st[i / 4][i % 4];
        }
        qc[c] = f32_to_chunk<T>(y);
      }
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


  float m_run = kNegInf;  // running max, log2 domain (identical in both halves)
  float l_run = 0.f;      // running sum over this lane half's keys
  f32x16 acc[NDT];
#pragma unroll
  for (int i = 0; i < NDT; ++i) acc[i] = (f32x16)(0.f);

  // c2 = |scale| * log2(e), kept strictly positive so a masked score (-inf)
  // always gives exp2(-inf * c2 - m) = 0 (sm_scale = 0 then yields the mean of
  // the valid V rows up to a ~1e-30 relative perturbation of the weights).
  const float c2 = fmaxf(fabsf(p.scale_log2), 1e-30f);
  // Valid keys of this lane's query: key < lim (kv_len, and causal key <= q).
  const int lim = CAUSAL ? min(p.kv_len, qrow + 1) : p.kv_len;

  TrAddr<T, D> vta;
  vta.init(lane);

  // Software pipeline over 64-key blocks, K one block ahead of V:
  //   iteration j:  S_{j+1} = K_{j+1} Q^T (MFMA)  |  exp / sum / pack of S_j (VALU)
  //                 O^T += V_j^T P_j^T    (MFMA)  |  masked max of S_{j+1} (VALU)
  // so each MFMA group has independent VALU work beside it in the same wave.
  // LDS: kbuf[2] and vbuf[2]; iteration j reads K_{j+1} and V_j while K_{j+2}
  // (into K_j's buffer) and V_{j+1} (into V_{j-1}'s) stream in.
  char* const kbuf0 = smem;
  char* const vbuf0 = smem + 2 * G::BYTES;
  auto kbuf = [&](int j) { return kbuf0 + (j & 1) * G::BYTES; };
  auto vbuf = [&](int j) { return vbuf0 + (j & 1) * G::BYTES; };

  // Masked row max of a block's scores (log2 units); masked entries of s
  // become -inf. lane half hh holds keys kv0 + 32hh + 16t + r.
  auto block_max = [&](f32x16* s, int kv0) -> float {
    const int rel = lim - kv0 - 32 * hh;
    float mx = kNegInf;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[t][r] = (16 * t + r < rel) ? s[t][r] : kNegInf;
        mx = fmaxf(mx, s[t][r]);
      }
    return wave_xor32_max(mx) * c2;
  };
  // Lazy rescale: the reference m_run only moves when some row's max grows
  // by more than 8 (log2 units), so p = 2^(x - m) stays below 2^8 and the O
  // rescale is rare; l and acc share the reference, so o is unchanged.
  auto update_max = [&](float mx) {
    const float m_cand = fmaxf(m_run, mx);
    if (__any(m_cand > m_run + 8.f)) {
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_cand);
#pragma unroll
      for (int i = 0; i < NDT; ++i) acc[i] *= alpha;
      l_run *= alpha;
      m_run = m_cand;
    }
  };
  // exp2 of a block's (masked) scores against m_run, summed into l_run and
  // packed as the B operand of O^T += V^T P^T.
  auto block_exp = [&](f32x16* s, Frag* pfr) {
    float rs = 0.f;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[t][r] = __builtin_amdgcn_exp2f(fmaf(s[t][r], c2, -m_run));
        rs += s[t][r];
      }
    l_run += rs;
    pack_frags<T>(s[0], s[1], pfr);
  };

  f32x16 s_cur[2];
  if (nblk > 0) {
    dma_wait();
    __syncthreads();
    s_cur[0] = (f32x16)(0.f);
    s_cur[1] = (f32x16)(0.f);
    mfma_nat<T, D>(kbuf(0), l32, hh, qf, s_cur[0], s_cur[1]);
    __syncthreads();  // every wave is done with K_0 before K_2 overwrites it
    update_max(block_max(s_cur, 0));
  }

  // 16-bit: per-lane max of the latest S block, reduced and applied at the
  // start of the next iteration (or before the last block's exp).
  float mx_carry = kNegInf;

  // Iteration j masks block j + 1. Blocks [0, n_plain) need no mask for any
  // row of the workgroup (below the causal diagonal, inside kv_len), so the
  // iterations run in two straight-line loops: plain max, then masked max.
  int n_plain = min(nblk, p.kv_len / BN);
  if constexpr (CAUSAL) n_plain = min(n_plain, (q0 + 1) / BN);

  // par = j & 1 as a compile-time constant: the LDS buffer addresses of an
  // iteration are then fixed and fold into the read instructions' offsets.
  auto iter = [&](auto masked, int j, auto par) __attribute__((always_inline)) {
    constexpr int P = decltype(par)::value;
    char* const kcur = kbuf0 + (1 - P) * G::BYTES;  // K_{j+1}
    char* const vcur = vbuf0 + P * G::BYTES;        // V_j
    const int kv1 = (j + 1) * BN;
    // DMA of K_{j+2} (into K_j's buffer) and V_{j+1} (into V_{j-1}'s buffer);
    // both were last read before the barrier that ended iteration j-1.
    // 16-bit: one load per MFMA slot of the S sequence below, not a burst:
    // a wave blocked on a full vector-memory queue issues no MFMAs either.
    char* const kdst = kbuf0 + P * G::BYTES;
    char* const vdst = vbuf0 + (1 - P) * G::BYTES;
    const bool k_next = j + 2 < nblk;
    const i32x4 kd = TileDma<T, D>::pinned_at_row(krs, kv1 + BN);
    const i32x4 vd = TileDma<T, D>::pinned_at_row(vrs, kv1);
    auto dma_part = [&](int i) __attribute__((always_inline)) {
      constexpr int PT = TileDma<T, D>::PER_T;
      if (i < PT) {
        if (k_next) dma.load_part(kd, i, kdst);
      } else if (i < 2 * PT) {
        dma.load_part(vd, i - PT, vdst);
      }
    };
    if constexpr (sizeof(T) != 2) {
      if (k_next) dma.load(krs, kv1 + BN, kdst);
      dma.load(vrs, kv1, vdst);
      __builtin_amdgcn_sched_barrier(0);
    }

    f32x16 s_nxt[2];
    s_nxt[0] = (f32x16)(0.f);
    s_nxt[1] = (f32x16)(0.f);
    Frag pfr[PF];
    float mx = kNegInf;
    if constexpr (sizeof(T) == 2) {
      // S_{j+1} MFMAs with the max update of S_j beside them, then
      // O^T += V_j^T P_j with the exp/sum/pack of S_j and the per-lane max of
      // S_{j+1} (32 / NV2 values per slot) beside it.
      constexpr int NV1 = G::CPR;
      constexpr int NV2 = 4 * NDT, VPS2 = 32 / NV2;
      // The row sum adds the float32 P (flash_attention.py:127-131: l from
      // the unrounded p; only the P.V operand is rounded).
      uint32_t pw[16];
      float rs = 0.f;
      // Slots 0-1 of the S sequence: finish the max of S_j (its per-lane part
      // was taken beside the previous iteration's P.V MFMAs) and update m.
      // The 16 exp pairs of S_j: kSPairs beside the S MFMAs, the rest beside
      // the P.V MFMAs: P.V MFMA k reads fragment k / NDT, so fragment f's four
      // pairs run in slots [(f - 1) NDT, f NDT) and it is packed in the last
      // of them, before its first MFMA. With the
      // exp work out of the S sequence its MFMAs issue back to back while the
      // max reduction and m update resolve: 4 of 16 pairs there measured
      // 3.8% faster at config 3 than all 16 (same box, bit-identical: the
      // row sum adds the pairs in the same order).
      constexpr int kSPairs = 4;
      static_assert(kSPairs >= 4 && kSPairs % 4 == 0 && kSPairs <= 16,
                    "fragment 0 is packed before the P.V sequence; f >= 1 in slot (f - 1) NDT + (3 NDT) / 4 < f NDT");
      float mxr = kNegInf;
      auto exp_pair = [&](int pr) __attribute__((always_inline)) {
        const int v = 2 * pr;  // value v = tile v / 16, register v % 16
        const float x0 = __builtin_amdgcn_exp2f(fmaf(s_cur[v >> 4][v & 15], c2, -m_run));
        const float x1 = __builtin_amdgcn_exp2f(fmaf(s_cur[v >> 4][(v & 15) + 1], c2, -m_run));
        pw[pr] = pack2<T>(x0, x1);
        rs += x0 + x1;
        // keeps the sum here: consumed only after the sequence, it would
        // otherwise sink to the end and hold every exp result live
        asm volatile("" : "+v"(rs));
      };
      mfma_nat_il<T, D>(kcur, l32, hh, qf, s_nxt[0], s_nxt[1], [&](int i) {
        dma_part(i);
        if (i == 0) {
          mxr = wave_xor32_max(mx_carry) * c2;
        } else if (i == 1) {
          update_max(mxr);
        } else {
#pragma unroll
          for (int pr = ((i - 2) * kSPairs) / (NV1 - 2); pr < ((i - 1) * kSPairs) / (NV1 - 2); ++pr) exp_pair(pr);
        }
      });
#pragma unroll
      for (int f = 0; f < kSPairs / 4; ++f)
        pfr[f] = __builtin_bit_cast(Frag, (u32x4){pw[4 * f], pw[4 * f + 1], pw[4 * f + 2], pw[4 * f + 3]});
      const int rel = lim - kv1 - 32 * hh;
      mfma_trn_il<T, D>(vcur, vta, pfr, acc, [&](int i) {
#pragma unroll
        for (int pr = kSPairs; pr < 16; ++pr) {
          const int f = pr >> 2, q4 = pr & 3;
          if (i == (f - 1) * NDT + (q4 * NDT) / 4) {
            exp_pair(pr);
            if (q4 == 3)
              pfr[f] = __builtin_bit_cast(Frag, (u32x4){pw[4 * f], pw[4 * f + 1], pw[4 * f + 2], pw[4 * f + 3]});
          }
        }
#pragma unroll
        for (int e = 0; e < VPS2; ++e) {
          const int v = i * VPS2 + e;
          float x = s_nxt[v >> 4][v & 15];
          if constexpr (decltype(masked)::value) {
            x = (v < rel) ? x : kNegInf;
            s_nxt[v >> 4][v & 15] = x;
          }
          mx = fmaxf(mx, x);
        }
        asm volatile("" : "+v"(mx));  // keeps the max beside its MFMA (see rs)
      });
      l_run += rs;
      mx_carry = mx;
    } else {
      mfma_nat<T, D>(kcur, l32, hh, qf, s_nxt[0], s_nxt[1]);
      block_exp(s_cur, pfr);
      mfma_trn<T, D>(vcur, lane, vta, pfr, acc);
      update_max(block_max(s_nxt, kv1));
    }
    s_cur[0] = s_nxt[0];
    s_cur[1] = s_nxt[1];

    dma_wait();
    __syncthreads();
  };
  // Iterations [0, jend) in pairs (even, odd), so each copy's buffers are fixed.
  using Even = std::integral_constant<int, 0>;
  using Odd = std::integral_constant<int, 1>;
  int j = 0;
  auto run = [&](auto masked, int jend) __attribute__((always_inline)) {
    if ((j & 1) && j < jend) iter(masked, j++, Odd{});
    for (; j + 1 < jend; j += 2) {
      iter(masked, j, Even{});
      iter(masked, j + 1, Odd{});
    }
    if (j < jend) iter(masked, j++, Even{});
  };
  run(std::false_type{}, min(n_plain, nblk) - 1);
  run(std::true_type{}, nblk - 1);

  if (nblk > 0) {
    if constexpr (sizeof(T) == 2) update_max(wave_xor32_max(mx_carry) * c2);
    Frag pfr[PF];
    block_exp(s_cur, pfr);
    mfma_trn<T, D>(vbuf(nblk - 1), lane, vta, pfr, acc);
  }

  // ---- finalize: o = acc / l, lse = m ln2 + ln l ---------------------------
  const float l_tot = wave_xor32_sum(l_run);
  if (qrow < p.Sq) {
    // one correctly rounded reciprocal, then multiplies (within 1.5 ulp of
    // acc / l, instead of 64 full divisions per lane)
    const float inv = 1.f / ((l_tot == 0.f) ? 1.f : l_tot);
    T* orow = static_cast<T*>(p.o) + ((int64_t)(b * p.Hq + h) * p.Sq + qrow) * D;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d0 = 32 * dt + 8 * r4 + 4 * hh;
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = acc[dt][4 * r4 + e] * inv;
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

// Row rotation: the K prologue of the fused-RoPE forward and pf_rope. A
// thread owns one 16-byte chunk of the first half of a row position `pos`
// together with its partner chunk D/2 further, loads that position's table
// values once and applies them to the same chunks of kHeadsPerThread rows
// (one per (batch, head), all at `pos`), rounding once to T. Rows at or past
// kv_len are not touched (the attention kernel never reads them). With halves
// x1 = x[:D/2], x2 = x[D/2:] and table halves c1, c2, s1, s2 of row pos:
//   forward (fused_rope.py:43-50, :75-78: x*cos + rotate_half(x)*sin)
//     y1 = x1 c1 - x2 s1,  y2 = x2 c2 + x1 s2;
//   inverse = the transpose of that linear map (the VJP of the forward one,
//   exact for any table, also when the halves of a table row differ)
//     y1 = x1 c1 + x2 s2,  y2 = x2 c2 - x1 s1.
// Consecutive threads take consecutive chunks, then positions, so each
// (batch, head)'s rows are read and written contiguously.
constexpr int kHeadsPerThread = 4;

template <typename T, int D, bool INVERSE>
__global__ __launch_bounds__(256) void pf_rope_rotate_k_kernel(const T* __restrict__ k, T* __restrict__ out,
                                                               const float* __restrict__ cosb,
                                                               const float* __restrict__ sinb, int Sk,
                                                               int kv_len, int n_bh, int64_t n_items) {
  constexpr int EPC = 16 / (int)sizeof(T);
  constexpr int HC = D / 2 / EPC;  // chunks per half row
  const int64_t item = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (item >= n_items) return;
  const int pc = (int)(item % HC);
  const int64_t rr = item / HC;  // (head group, position < kv_len)
  const int pos = (int)(rr % kv_len);
  const int bh0 = (int)(rr / kv_len) * kHeadsPerThread;
  const int nh = min(kHeadsPerThread, n_bh - bh0);
  const float* cs = cosb + (int64_t)pos * D + pc * EPC;
  const float* sn = sinb + (int64_t)pos * D + pc * EPC;
  float c1[EPC], c2[EPC], s1[EPC], s2[EPC];
#pragma unroll
  for (int e = 0; e < EPC; ++e) {
    c1[e] = cs[e];
    c2[e] = cs[D / 2 + e];
    s1[e] = sn[e];
    s2[e] = sn[D / 2 + e];
  }
  u32x4 lo[kHeadsPerThread], hi[kHeadsPerThread];
#pragma unroll
  for (int j = 0; j < kHeadsPerThread; ++j) {
    if (j < nh) {
      const T* src = k + ((int64_t)(bh0 + j) * Sk + pos) * D + pc * EPC;
      lo[j] = ldg16_nt(src);  // each row is read once
      hi[j] = ldg16_nt(src + D / 2);
    }
  }
#pragma unroll
  for (int j = 0; j < kHeadsPerThread; ++j) {
    if (j < nh) {
      float a[EPC], bb[EPC], ra[EPC], rb[EPC];
      chunk_to_f32<T>(lo[j], a);
      chunk_to_f32<T>(hi[j], bb);
#pragma unroll
      for (int e = 0; e < EPC; ++e) {
        if constexpr (INVERSE) {
          ra[e] = a[e] * c1[e] + bb[e] * s2[e];
          rb[e] = bb[e] * c2[e] - a[e] * s1[e];
        } else {
          ra[e] = a[e] * c1[e] - bb[e] * s1[e];
          rb[e] = bb[e] * c2[e] + a[e] * s2[e];
        }
      }
      T* dst = out + ((int64_t)(bh0 + j) * Sk + pos) * D + pc * EPC;
      stg16(dst, f32_to_chunk<T>(ra));
      stg16(dst + D / 2, f32_to_chunk<T>(rb));
    }
  }
}

template <typename T, int D>
hipError_t launch_typed(const FwdParams& p, bool causal, bool rope, hipStream_t st) {
  const dim3 grid(work_tail_grid(p.tail, p.n_work)), block(256);
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
  if constexpr (sizeof(T) == 2)
    if (head_dim == 256) return launch_typed<T, 256>(p, causal, rope, st);
  return hipErrorInvalidValue;
}

template <typename T, int D>
hipError_t rotate_typed(const void* k, void* out, const float* cs, const float* sn, int B, int Hkv, int Sk,
                        int kv_len, bool inverse, hipStream_t st) {
  constexpr int HC = D / 2 / (16 / (int)sizeof(T));
  const int n_bh = B * Hkv;
  const int64_t n_items = (int64_t)((n_bh + kHeadsPerThread - 1) / kHeadsPerThread) * kv_len * HC;
  if (n_items == 0) return hipSuccess;
  const dim3 grid((unsigned)((n_items + 255) / 256)), block(256);
  if (inverse)
    hipLaunchKernelGGL((pf_rope_rotate_k_kernel<T, D, true>), grid, block, 0, st, static_cast<const T*>(k),
                       static_cast<T*>(out), cs, sn, Sk, kv_len, n_bh, n_items);
  else
    hipLaunchKernelGGL((pf_rope_rotate_k_kernel<T, D, false>), grid, block, 0, st, static_cast<const T*>(k),
                       static_cast<T*>(out), cs, sn, Sk, kv_len, n_bh, n_items);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_rope_rotate_k(const void* k, void* k_out, const float* cos, const float* sin, int B,
                                int Hkv, int Sk, int kv_len, int dtype, int head_dim, hipStream_t stream,
                                bool inverse) {
  const bool inv = inverse;
  if (head_dim == 128) {
    if (dtype == kF32) return rotate_typed<float, 128>(k, k_out, cos, sin, B, Hkv, Sk, kv_len, inv, stream);
    if (dtype == kBF16) return rotate_typed<bf16_t, 128>(k, k_out, cos, sin, B, Hkv, Sk, kv_len, inv, stream);
    if (dtype == kF16) return rotate_typed<f16_t, 128>(k, k_out, cos, sin, B, Hkv, Sk, kv_len, inv, stream);
  } else if (head_dim == 64) {
    if (dtype == kF32) return rotate_typed<float, 64>(k, k_out, cos, sin, B, Hkv, Sk, kv_len, inv, stream);
    if (dtype == kBF16) return rotate_typed<bf16_t, 64>(k, k_out, cos, sin, B, Hkv, Sk, kv_len, inv, stream);
    if (dtype == kF16) return rotate_typed<f16_t, 64>(k, k_out, cos, sin, B, Hkv, Sk, kv_len, inv, stream);
  } else if (head_dim == 256) {
    if (dtype == kBF16) return rotate_typed<bf16_t, 256>(k, k_out, cos, sin, B, Hkv, Sk, kv_len, inv, stream);
    if (dtype == kF16) return rotate_typed<f16_t, 256>(k, k_out, cos, sin, B, Hkv, Sk, kv_len, inv, stream);
  }
  return hipErrorInvalidValue;
}

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
