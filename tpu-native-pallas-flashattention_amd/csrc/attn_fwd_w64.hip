// Forward prefill attention for gfx950, 16-bit inputs, D = 128: the wide
// variant with 64 query rows per wave (with optional fused RoPE on Q; K
// arrives rotated by pf_rope_rotate_k_kernel). Opt-in (the host selects it
// only with PF_FWD_ROWS_PER_WAVE=64): it computes the same results as the
// 32-row kernel of attn_fwd.hip but measures slower at the headline shapes
// (one workgroup per CU exposes every barrier and every work item's
// prologue and epilogue; the 32-row kernel's two workgroups per CU cover
// each other's).
//
// Replaces the same reference calls as attn_fwd.hip (flash_attention.py:162-227,
// kernel :61-159; fused_rope.py:183-213, kernel :53-113) with the same
// semantics and the same online-softmax arithmetic; only the tiling differs.
//
// Why a second tiling: with 32 query rows per wave every 16-byte K or V^T
// operand a lane reads from LDS feeds exactly one 32x32x16 MFMA, and issuing
// and waiting on those reads, not the matrix cores, bounds the loop (an MFMA
// + LDS-read probe of that shape reaches 62% of peak at 2 workgroups per CU;
// the LDS itself shows no back-pressure). Here each wave
// owns two 32-row query tiles, so every K chunk and every V^T fragment read
// feeds two MFMAs (the same probe: 77% of peak at 1 workgroup per CU).
// The price is one wave per SIMD: 128 O accumulators (AGPRs), 64 Q registers
// (AGPRs: the S MFMAs take Q as an AGPR B operand), 2 x 64 S registers and
// the operand rings (VGPRs) fill the 512-entry register file, so the MFMA /
// VALU overlap must come from one instruction stream. The block loop is one
// fenced sequence of 64 MFMA slots per 64-key block:
//   slots  0..31  S_{j+1} = K_{j+1} Q^T  | m update; exp/sum/pack of S_j
//                                          for P.V step 0 and half of step 1
//   slots 32..63  O^T += V_j^T P_j^T     | exp/sum/pack for the rest; per-lane
//                                          max of S_{j+1}
// The exp work is software-pipelined over consecutive slots (exp_slot), and
// every LDS operand read is issued a few slots ahead of its MFMA -- also
// across the two phases and across the barrier that ends the block, so that
// no LDS latency bubble follows the barrier. Blocks crossing the causal
// diagonal or kv_len are masked after the sequence, with their max taken
// again.
//
// LDS: 4 K buffers and 4 V buffers (128 KB). Iteration j stages V_{j+2} and
// K_{j+4} by DMA and, before its closing barrier, waits only for the tiles
// staged one iteration earlier (vmcnt(8)): every tile load gets a full
// iteration of latency, and K_{j+2} is already published when iteration j
// reads ahead its first chunks.
#include "pf_common.hpp"
#include "pf_kernels.hpp"
#include "pf_tiles.hpp"

#include <type_traits>

namespace pf {

namespace {

// S MFMA with the float32 accumulator in VGPRs and the B operand (Q) in
// AGPRs, as inline assembly (the builtin cannot place an operand in AGPRs).
// Wait states the compiler cannot see inside the asm: s_nop 1 covers a VALU
// write of an operand (v_accvgpr_write of Q, a VALU write of the
// accumulator) just before; the results are read only after vfence4 below.
template <typename T>
struct MfmaVA;
template <>
struct MfmaVA<bf16_t> {
  __device__ static inline void first(f32x16& s, bf16x8 a, bf16x8 b) {
    asm("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(s) : "v"(a), "a"(b));
  }
  __device__ static inline void run(f32x16& s, bf16x8 a, bf16x8 b) {
    asm("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(s) : "v"(a), "a"(b));
  }
};
template <>
struct MfmaVA<f16_t> {
  __device__ static inline void first(f32x16& s, f16x8 a, f16x8 b) {
    asm("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, 0" : "=&v"(s) : "v"(a), "a"(b));
  }
  __device__ static inline void run(f32x16& s, f16x8 a, f16x8 b) {
    asm("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(s) : "v"(a), "a"(b));
  }
};

// max of two floats as one v_max_f32 (the MFMA results of the asm above are
// opaque to the compiler, which would otherwise canonicalize every input with
// an extra v_max_f32 first).
__device__ inline float fmax_raw(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

__device__ inline float fmax3_raw(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// Software pipeline of the exp work: pair P (0..31) of S_j is P = 8 c + 4 qt + i,
// the values v = 8 c + 2 i, 8 c + 2 i + 1 of query tile qt (key tile v / 16,
// register v % 16), i.e. the P^T fragment of PV step c. Stage A (two FMAs)
// runs in slot exp_slot(P), stage B (two exp2) one slot later, stage C (pack,
// pair sum) two, stage D (row-sum add) three: no VALU op waits on another of
// its own slot. The first kExpS pairs run beside the S MFMAs, the rest beside
// the P.V MFMAs, each finished (stage C) before the first P.V MFMA that reads
// its fragment (kExpOrderOk). The P.V phase also carries the max of S_{j+1},
// so the S phase takes fewer pairs: 12 of 32 measured 3% faster than 24 at
// config 3 and 2% faster than 16 (same box, bit-identical); 4 breaks the
// ordering.
constexpr int kExpS = 12;
__host__ __device__ constexpr int exp_slot(int P) {
  return P < kExpS ? 2 + (P * 26) / kExpS : 32 + ((P - kExpS) * 22) / (32 - kExpS);
}
// Pair P feeds P.V step c = P / 8 for query tile qt = (P / 4) % 2, whose
// first MFMA is slot 32 + 8 c + qt; stage D must fit in the sequence.
__host__ __device__ constexpr bool kExpOrderOk() {
  for (int P = 0; P < 32; ++P) {
    if (exp_slot(P) + 2 >= 32 + 8 * (P >> 3) + ((P >> 2) & 1)) return false;
    if (exp_slot(P) + 3 > 63 || (P > 0 && exp_slot(P) < exp_slot(P - 1))) return false;
  }
  return true;
}
static_assert(kExpOrderOk(), "every P fragment is packed before its first P.V MFMA");
// First pair whose stage A slot is >= slot (exp_slot is non-decreasing), so
// the pairs whose stage A runs in slot s are [pair_lo(s), pair_lo(s + 1)).
__host__ __device__ constexpr int pair_lo(int slot) {
  int P = 0;
  while (P < 32 && exp_slot(P) < slot) ++P;
  return P;
}

// Fences for the results of the asm MFMAs above. The compiler cannot see
// that those instructions write their outputs late, so any read it makes of
// an output -- including register copies it inserts on its own, e.g. where
// two paths meet -- must come after a fence that takes the values as tied
// operands (ordered after the MFMAs by data dependence) and waits 16 states.
__device__ inline void vfence4(f32x16& a, f32x16& b, f32x16& c, f32x16& d) {
  asm volatile("s_nop 7\n\ts_nop 7" : "+v"(a), "+v"(b), "+v"(c), "+v"(d));
}
__device__ inline void afence8(f32x16 (&x)[2][4]) {
  asm volatile("s_nop 7\n\ts_nop 7"
               : "+a"(x[0][0]), "+a"(x[0][1]), "+a"(x[0][2]), "+a"(x[0][3]), "+a"(x[1][0]), "+a"(x[1][1]),
                 "+a"(x[1][2]), "+a"(x[1][3]));
}

template <typename T, bool CAUSAL, bool ROPE, int LC = 2, int LP = 4>
__global__ __launch_bounds__(256, 1) void pf_attn_fwd_w64_kernel(FwdParams p) {
  constexpr int D = 128;
  using MF = Mfma32<T>;
  using Frag = typename MF::Frag;
  using G = Tile<T, D>;
  using DMA = TileDma<T, D>;
  using VA = MfmaVA<T>;
  static_assert(sizeof(T) == 2, "16-bit operands");
  constexpr int BN = 64;       // keys per block
  constexpr int HALF = D / 2;
  constexpr int EPC = G::EPC;  // 8 elements per 16-byte chunk
  constexpr int NCH = HALF / EPC;  // 8 chunks (= MFMA steps of S) per lane half
  constexpr int NDT = D / 32;      // 4 column blocks of O^T
  constexpr int NKB = 4, NVB = 4;  // K and V buffers
  constexpr int RB = G::RB;
  constexpr int PT = DMA::PER_T;   // DMA loads per tile per wave (4)
  static_assert(LP % 2 == 0 && LP >= 2 && LC >= 1 && 2 * LC <= 32 - 2, "read leads");

  __shared__ __attribute__((aligned(16))) char smem[(NKB + NVB) * G::BYTES];
  char* const kb0 = smem;
  char* const vb0 = smem + NKB * G::BYTES;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int hh = lane >> 5;
  const int l32 = lane & 31;

  // work item = (query block, batch, kv head, head group); the waves split
  // into hpw heads x (4 / hpw) 64-row slices.
  int b, kvh, hg, qblk;
  fwd_work_item(blockIdx.x, p, b, kvh, hg, qblk);
  const int wph = 4 / p.hpw;
  const int h = kvh * p.g + hg * p.hpw + wv / wph;
  const int q0 = qblk * p.rpw;
  const int wq0 = q0 + 64 * (wv % wph);

  const T* Qb = static_cast<const T*>(p.q) + (int64_t)(b * p.Hq + h) * p.Sq * D;
  const T* Kb = static_cast<const T*>(p.k) + (int64_t)(b * p.Hkv + kvh) * p.Sk * D;
  const T* Vb = static_cast<const T*>(p.v) + (int64_t)(b * p.Hkv + kvh) * p.Sk * D;

  int kv_end = p.kv_len;
  if constexpr (CAUSAL) kv_end = min(kv_end, min(q0 + p.rpw, p.Sq));
  const int nblk = (kv_end + BN - 1) / BN;
  // The buffer resources end at the last block this item uses (and at
  // kv_len): the loop's look-ahead loads past it fetch nothing and write
  // zeros, and rows past kv_len are never read from memory.
  const uint32_t kv_bytes = (uint32_t)min(p.kv_len, nblk * BN) * (uint32_t)RB;
  const i32x4 krs = make_desc(Kb, kv_bytes);
  const i32x4 vrs = make_desc(Vb, kv_bytes);
  DMA dma;
  dma.init(tid);
  if (nblk > 0) {
#pragma unroll
    for (int t = 0; t < 4; ++t) dma.load(krs, t * BN, kb0 + t * G::BYTES);
    dma.load(vrs, 0, vb0);
    dma.load(vrs, BN, vb0 + G::BYTES);
  }

  // ---- Q fragments (B operand of S^T): query tile qt, lane holds
  // Q[wq0 + 32 qt + l32][hh*HALF, +HALF).
  Frag qf[2][NCH];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int qrow = wq0 + 32 * qt + l32;
    u32x4 qc[NCH];
    if (qrow < p.Sq) {
      const T* qr = Qb + (int64_t)qrow * D;
      if constexpr (ROPE) {
        const float* cs = p.q_cos + (int64_t)qrow * D;
        const float* sn = p.q_sin + (int64_t)qrow * D;
        const float sgn = hh ? 1.f : -1.f;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
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
        for (int c = 0; c < NCH; ++c) qc[c] = ldg16(qr + hh * HALF + c * EPC);
      }
    } else {
#pragma unroll
      for (int c = 0; c < NCH; ++c) qc[c] = (u32x4){0u, 0u, 0u, 0u};
    }
    // a negative scale is applied as |scale| on -Q (exact sign flips)
    if (p.scale_log2 < 0.f) {
#pragma unroll
      for (int c = 0; c < NCH; ++c) qc[c] ^= (u32x4){0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u};
    }
    // Move Q to AGPRs for good: the asm output is an AGPR-class value, and
    // every later use (the S MFMAs' "a" operand) keeps it there.
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const Frag qv = __builtin_bit_cast(Frag, qc[c]);
      asm volatile("; q to agpr" : "=a"(qf[qt][c]) : "0"(qv));
    }
  }

  float m_run[2] = {kNegInf, kNegInf};  // running max, log2 domain
  float l_run[2] = {0.f, 0.f};          // running sum over this lane half's keys
  f32x16 acc[2][NDT];                   // O^T, AGPRs
#pragma unroll
  for (int qt = 0; qt < 2; ++qt)
#pragma unroll
    for (int i = 0; i < NDT; ++i) acc[qt][i] = (f32x16)(0.f);

  const float c2 = fmaxf(fabsf(p.scale_log2), 1e-30f);
  int lim[2];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) lim[qt] = CAUSAL ? min(p.kv_len, wq0 + 32 * qt + l32 + 1) : p.kv_len;

  TrAddr<T, D> vta;
  vta.init(lane);
  const int r0 = mfma_src_row(l32, 0), r1 = mfma_src_row(l32, 1);
  const int sw0 = tile_swz<G::CPR>(r0), sw1 = tile_swz<G::CPR>(r1);

  // K chunk c of both 32-row halves of a tile (natural A operands of S^T).
  // Chunk c of key tile kt (rows mfma_src_row(l32, kt)) of a K tile: the
  // natural A operand of S^T. The lane offset is recomputed at each read (one
  // XOR and one shift-add): kept as loop invariants the 16 offsets would hold
  // 16 more registers.
  auto kread = [&](const char* tile, int kt, int c) __attribute__((always_inline)) -> u32x4 {
    int x = (hh * NCH) ^ (kt ? sw1 : sw0);
    asm volatile("" : "+v"(x));
    return lds16(tile + (kt ? r1 : r0) * RB + 16 * (x ^ c));
  };
  // V^T fragment k = step c * NDT + column block dt (transposed A operand of O^T).
  auto vread = [&](const char* tile, int k) __attribute__((always_inline)) -> Frag {
    typedef short v4i16 __attribute__((ext_vector_type(4)));
    const int c = k / NDT, dt = k % NDT;
    v4i16 part[2];
#pragma unroll
    for (int r = 0; r < 2; ++r)
      part[r] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) v4i16*)(tile + vta.off[dt][r] + (8 * c + 4 * r) * RB));
    return __builtin_bit_cast(Frag, __builtin_shufflevector(part[0], part[1], 0, 1, 2, 3, 4, 5, 6, 7));
  };
  auto update_max = [&](int qt, float mx) __attribute__((always_inline)) {
    const float m_cand = fmaxf(m_run[qt], mx);
    // lazy rescale: the reference max only moves when a row's max grows by
    // more than 8 (log2 units), so p = 2^(x - m) stays below 2^8
    if (__any(m_cand > m_run[qt] + 8.f)) {
      const float alpha = __builtin_amdgcn_exp2f(m_run[qt] - m_cand);
#pragma unroll
      for (int i = 0; i < NDT; ++i) {
        agpr_fence(acc[qt][i]);
        acc[qt][i] *= alpha;
      }
      l_run[qt] *= alpha;
      m_run[qt] = m_cand;
    }
  };

  // S blocks alternate between two register sets: S_j lives in sset[j & 1].
  f32x16 sset[2][2][2];  // [set][key half kt][query tile qt]
  // ring of K chunks read ahead: chunk g = 8 kt + c of the current S tile in
  // kring[g % (LC + 1)]
  u32x4 kring[LC + 1];
  // per-lane (unreduced) max of the latest S block
  float mx_carry[2] = {kNegInf, kNegInf};

  if (nblk > 0) {
    dma_wait();
    __syncthreads();
    // S_0 and its masked max (reduced here; the loop carries it from then on)
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        const Frag a = __builtin_bit_cast(Frag, kread(kb0, kt, c));
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
          if (c == 0) VA::first(sset[0][kt][qt], a, qf[qt][c]);
          else VA::run(sset[0][kt][qt], a, qf[qt][c]);
        }
      }
    vfence4(sset[0][0][0], sset[0][0][1], sset[0][1][0], sset[0][1][1]);
    __syncthreads();  // every wave is done with K_0 before K_4 overwrites it
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      const int rel = lim[qt] - 32 * hh;
      float mx = kNegInf;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float x = (16 * kt + r < rel) ? sset[0][kt][qt][r] : kNegInf;
          sset[0][kt][qt][r] = x;
          mx = fmaxf(mx, x);
        }
      update_max(qt, wave_xor32_max(mx) * c2);
    }
    // read ahead the first chunks of K_1 (published by the first barrier)
#pragma unroll
    for (int g = 0; g < LC; ++g) kring[g] = kread(kb0 + G::BYTES, g / NCH, g % NCH);
  }

  int n_plain = min(nblk, p.kv_len / BN);
  if constexpr (CAUSAL) n_plain = min(n_plain, q0 / BN);

  // Iteration j (P = j % 4 at compile time, so every LDS buffer address folds
  // into the instructions' offsets): S_{j+1} and O += V_j^T P_j.
  auto iter = [&](int j, auto par) __attribute__((always_inline)) {
    constexpr int P = decltype(par)::value;
    char* const kcur = kb0 + ((P + 1) % NKB) * G::BYTES;   // K_{j+1}
    char* const knext = kb0 + ((P + 2) % NKB) * G::BYTES;  // K_{j+2} (read ahead)
    char* const vcur = vb0 + (P % NVB) * G::BYTES;         // V_j
    char* const kdst = kb0 + (P % NKB) * G::BYTES;         // K_{j+4} into K_j's buffer
    char* const vdst = vb0 + ((P + 2) % NVB) * G::BYTES;   // V_{j+2} into V_{j-2}'s buffer
    f32x16(&sc)[2][2] = sset[P & 1];        // S_j
    f32x16(&sn)[2][2] = sset[(P + 1) & 1];  // S_{j+1}
    const int kv1 = (j + 1) * BN;
    const i32x4 vd = DMA::at_row(vrs, (j + 2) * BN);
    const i32x4 kd = DMA::at_row(krs, (j + 4) * BN);

    uint32_t pw[32];     // packed P_j pairs, by pair index
    float ya[32][2];     // stage A results (exp2 arguments)
    float eb[32][2];     // stage B results (p)
    float tc[32];        // stage C results (pair sums)
    float rs[2] = {0.f, 0.f};
    float mxr[2];
    float mx[2] = {kNegInf, kNegInf};
    Frag pfr[2][4];
    Frag vring[LP / 2 + 1];

    static_for<64>([&](auto mc) __attribute__((always_inline)) {
      constexpr int m = decltype(mc)::value;
      // ---- LDS reads ahead of their MFMAs. S slot m uses K chunk
      // g = m / 2 (key tile g / 8, step g % 8) for query tiles 0 and 1.
      if constexpr (m < 32 && (m & 1) == 0 && (m >> 1) + LC < 2 * NCH) {
        constexpr int g = (m >> 1) + LC;
        kring[g % (LC + 1)] = kread(kcur, g / NCH, g % NCH);
      }
      if constexpr (m >= 32 - LP && m < 64 - LP && ((m + LP) & 1) == 0) {
        constexpr int k = (m + LP - 32) >> 1;
        vring[k % (LP / 2 + 1)] = vread(vcur, k);
      }
      if constexpr (m >= 64 - 2 * LC && (m & 1) == 0) {
        constexpr int g = (m - (64 - 2 * LC)) >> 1;  // chunk g of K_{j+2}
        kring[g % (LC + 1)] = kread(knext, g / NCH, g % NCH);
      }
      // ---- MFMA m
      if constexpr (m < 32) {
        constexpr int g = m >> 1, kt = g / NCH, c = g % NCH, qt = m & 1;
        const Frag a = __builtin_bit_cast(Frag, kring[g % (LC + 1)]);
        if constexpr (c == 0) VA::first(sn[kt][qt], a, qf[qt][c]);
        else VA::run(sn[kt][qt], a, qf[qt][c]);
      } else {
        constexpr int i = m - 32, k = i >> 1, qt = i & 1;
        constexpr int c = k / NDT, dt = k % NDT;
        MfmaAgpr<T>::run(acc[qt][dt], vring[k % (LP / 2 + 1)], pfr[qt][c]);
      }
      // ---- staging: V_{j+2} and K_{j+4}, one load per 4 slots
      if constexpr (m < 32 && (m & 3) == 3) {
        constexpr int u = m >> 2;
        if constexpr (u < PT) dma.load_part(vd, u, vdst);
        else dma.load_part(kd, u - PT, kdst);
      }
      // ---- VALU beside the MFMAs
      if constexpr (m == 0) {
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) mxr[qt] = wave_xor32_max(mx_carry[qt]) * c2;
      } else if constexpr (m == 1) {
        update_max(0, mxr[0]);
        update_max(1, mxr[1]);
      }
      // exp / sum / pack of S_j, software-pipelined (exp_slot): stage st of
      // the pairs whose stage A ran st slots ago
      auto stage = [&](auto pc, auto stc) __attribute__((always_inline)) {
        constexpr int P = decltype(pc)::value, st = decltype(stc)::value;
        constexpr int c = P >> 3, qt = (P >> 2) & 1, i = P & 3;
        constexpr int v = 8 * c + 2 * i, kt = v >> 4, r = v & 15;
        if constexpr (st == 0) {
          ya[P][0] = fmaf(sc[kt][qt][r], c2, -m_run[qt]);
          ya[P][1] = fmaf(sc[kt][qt][r + 1], c2, -m_run[qt]);
          asm volatile("" : "+v"(ya[P][0]), "+v"(ya[P][1]));
        } else if constexpr (st == 1) {
          eb[P][0] = __builtin_amdgcn_exp2f(ya[P][0]);
          eb[P][1] = __builtin_amdgcn_exp2f(ya[P][1]);
          asm volatile("" : "+v"(eb[P][0]), "+v"(eb[P][1]));
        } else if constexpr (st == 2) {
          pw[P] = pack2<T>(eb[P][0], eb[P][1]);
          tc[P] = eb[P][0] + eb[P][1];
          asm volatile("" : "+v"(pw[P]), "+v"(tc[P]));
          if constexpr (i == 3)  // the 4 pairs of this (step, query tile) are packed
            pfr[qt][c] = __builtin_bit_cast(Frag, (u32x4){pw[P - 3], pw[P - 2], pw[P - 1], pw[P]});
        } else {
          rs[qt] += tc[P];
          asm volatile("" : "+v"(rs[qt]));
        }
      };
      static_for<4>([&](auto stc) __attribute__((always_inline)) {
        constexpr int st = decltype(stc)::value;
        if constexpr (m >= st)
          static_for_range<pair_lo(m - st), pair_lo(m - st + 1)>(
              [&](auto pc) __attribute__((always_inline)) { stage(pc, stc); });
      });
      if constexpr (m == 31) vfence4(sn[0][0], sn[0][1], sn[1][0], sn[1][1]);  // S_{j+1} is read from here on
      if constexpr (m >= 32) {
        // per-lane max of S_{j+1}: 2 of its 64 values per slot, key tile 0
        // first (its last MFMA was slot 15)
        constexpr int vv = 2 * (m - 32), kt = vv >> 5, qt = (vv >> 4) & 1, r = vv & 15;
        mx[qt] = fmax3_raw(mx[qt], sn[kt][qt][r], sn[kt][qt][r + 1]);
        asm volatile("" : "+v"(mx[qt]));
      }
      __builtin_amdgcn_sched_barrier(0);
    });
    afence8(acc);  // O^T is carried to the next iteration (or the last block)
    l_run[0] += rs[0];
    l_run[1] += rs[1];
    // Block j + 1 crosses the causal diagonal or kv_len for some row of the
    // workgroup (only the last few blocks do): mask it and take the max again.
    if (j + 1 >= n_plain) {
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        const int rel = lim[qt] - kv1 - 32 * hh;
        float mm = kNegInf;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float x = (16 * kt + r < rel) ? sn[kt][qt][r] : kNegInf;
            sn[kt][qt][r] = x;
            mm = fmax_raw(mm, x);
          }
        mx[qt] = mm;
      }
    }
    mx_carry[0] = mx[0];
    mx_carry[1] = mx[1];
    // V_{j+1} and K_{j+3} (staged by the previous iteration) have landed;
    // this iteration's 2 x PT loads may still be in flight.
    wait_vm<2 * PT>();
    __syncthreads();
  };

  // All iterations in one loop, unrolled by 4 (the LDS buffer cycle), with an
  // exit after each copy.
  {
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    using P2 = std::integral_constant<int, 2>;
    using P3 = std::integral_constant<int, 3>;
    const int jend = nblk - 1;
    int j = 0;
    while (j < jend) {
      iter(j, P0{});
      if (++j >= jend) break;
      iter(j, P1{});
      if (++j >= jend) break;
      iter(j, P2{});
      if (++j >= jend) break;
      iter(j, P3{});
      ++j;
    }
  }

  // last block: m update, exp of S_{nblk-1}, O += V^T P (set index of
  // S_{nblk-1} as a compile-time constant, so the S sets stay in registers)
  auto last_block = [&](auto setc) __attribute__((always_inline)) {
    f32x16(&sc)[2][2] = sset[decltype(setc)::value];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) update_max(qt, wave_xor32_max(mx_carry[qt]) * c2);
    Frag pfr[2][4];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      uint32_t pw[16];
      float rs = 0.f;
#pragma unroll
      for (int pr = 0; pr < 16; ++pr) {
        const int v = 2 * pr;
        const float x0 = __builtin_amdgcn_exp2f(fmaf(sc[v >> 4][qt][v & 15], c2, -m_run[qt]));
        const float x1 = __builtin_amdgcn_exp2f(fmaf(sc[v >> 4][qt][(v & 15) + 1], c2, -m_run[qt]));
        pw[pr] = pack2<T>(x0, x1);
        rs += x0 + x1;
      }
      l_run[qt] += rs;
#pragma unroll
      for (int f = 0; f < 4; ++f)
        pfr[qt][f] = __builtin_bit_cast(Frag, (u32x4){pw[4 * f], pw[4 * f + 1], pw[4 * f + 2], pw[4 * f + 3]});
    }
    const char* vl = vb0 + ((nblk - 1) % NVB) * G::BYTES;
#pragma unroll
    for (int k = 0; k < 4 * NDT; ++k) {
      const Frag a = vread(vl, k);
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) MfmaAgpr<T>::run(acc[qt][k % NDT], a, pfr[qt][k / NDT]);
    }
    afence8(acc);
  };
  if (nblk > 0) {
    if ((nblk - 1) & 1) last_block(std::integral_constant<int, 1>{});
    else last_block(std::integral_constant<int, 0>{});
  }
  // look-ahead loads of the last iterations still write LDS
  dma_wait();

  // ---- finalize: o = acc / l, lse = m ln2 + ln l ---------------------------
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
#pragma unroll
    for (int i = 0; i < NDT; ++i) agpr_fence(acc[qt][i]);
    const int qrow = wq0 + 32 * qt + l32;
    const float l_tot = wave_xor32_sum(l_run[qt]);
    if (qrow < p.Sq) {
      // one correctly rounded reciprocal, then multiplies
      const float inv = 1.f / ((l_tot == 0.f) ? 1.f : l_tot);
      T* orow = static_cast<T*>(p.o) + ((int64_t)(b * p.Hq + h) * p.Sq + qrow) * D;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const int d0 = 32 * dt + 8 * r4 + 4 * hh;
          typedef T v4 __attribute__((ext_vector_type(4)));
          v4 x;
#pragma unroll
          for (int e = 0; e < 4; ++e) x[e] = Elem<T>::from_f32(acc[qt][dt][4 * r4 + e] * inv);
          *reinterpret_cast<v4*>(orow + d0) = x;
        }
      if (hh == 0 && p.lse != nullptr)
        p.lse[(int64_t)(b * p.Hq + h) * p.Sq + qrow] = (l_tot == 0.f) ? 0.f : m_run[qt] * kLn2 + logf(l_tot);
    }
  }
}

template <typename T>
hipError_t launch_w64_typed(const FwdParams& p, bool causal, bool rope, hipStream_t st) {
  const dim3 grid(p.n_work), block(256);
  if (causal) {
    if (rope) hipLaunchKernelGGL((pf_attn_fwd_w64_kernel<T, true, true>), grid, block, 0, st, p);
    else hipLaunchKernelGGL((pf_attn_fwd_w64_kernel<T, true, false>), grid, block, 0, st, p);
  } else {
    if (rope) hipLaunchKernelGGL((pf_attn_fwd_w64_kernel<T, false, true>), grid, block, 0, st, p);
    else hipLaunchKernelGGL((pf_attn_fwd_w64_kernel<T, false, false>), grid, block, 0, st, p);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_attn_fwd_w64(const FwdParams& p, int dtype, bool causal, bool rope, hipStream_t stream) {
  if (p.rows_per_wave != 64) return hipErrorInvalidValue;
  switch (dtype) {
    case kBF16: return launch_w64_typed<bf16_t>(p, causal, rope, stream);
    case kF16: return launch_w64_typed<f16_t>(p, causal, rope, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace pf
